"""CPU oracle for the HashPrune reducer (oracle/tessa_hashprune.c), pinned.

Reference (shear-core/src/algorithm/pipnn/): the reservoir KATs of
hash_prune.rs:4803-4875, the total order :2094-2106 and insert :1333-1453,
the spill reducer's stream insertion spill_hashprune.rs:2686-2719 / :3203-3221.
Independent checks: a brute-force restatement (each hash's best candidate,
then the l_max best of those, listed by ascending hash) and invariance under
shuffles of the record stream.
"""
import numpy as np
import pytest

from oracle import pyoracle as O


def recs(rows):
    """[(src, dst, hash, dist)] -> EDGE_DTYPE records."""
    out = np.zeros(len(rows), O.EDGE_DTYPE)
    for i, (s, d, h, x) in enumerate(rows):
        out[i] = (s, d, h, 0, x)
    return out


def one_point(l_max, cands):
    t, hs, d, cnt = O.hashprune_reduce(1, l_max, recs([(0, c, h, x) for c, h, x in cands]))
    return t[0, :cnt[0]], hs[0, :cnt[0]], d[0, :cnt[0]]


def bf16(x):
    return np.array([x], np.float32).view(np.uint32)[0] >> 16


def test_kat_full_path_exact_distance_for_farthest_replacement():
    # hash_prune.rs:4803-4819: both candidates share one BF16 bucket
    better, worse = (10, 10, 66_703.0), (20, 20, 66_763.0)
    assert bf16(better[2]) == bf16(worse[2])
    t, _, _ = one_point(2, [(1, 1, 10.0), worse, better])
    assert sorted(t.tolist()) == [1, 10]


def test_kat_same_hash_collision_exact_distance():
    # hash_prune.rs:4821-4836
    t, _, _ = one_point(4, [(20, 7, 66_763.0), (10, 7, 66_703.0)])
    assert sorted(t.tolist()) == [10]


def test_kat_nearer_inside_legacy_epsilon_band():
    # hash_prune.rs:4838-4845 and :4847-4854
    t, _, _ = one_point(1, [(30, 30, 1.0), (20, 20, 1.0 + 1.5e-5)])
    assert t.tolist() == [30]
    t, _, _ = one_point(4, [(30, 7, 1.0), (20, 7, 1.0 + 1.5e-5)])
    assert t.tolist() == [30]


def test_kat_permutation_independent_epsilon_cycle():
    # hash_prune.rs:4856-4875
    cands = [(2, 7, 0.0), (1, 7, 1.5e-5), (0, 7, 3.0e-5)]
    for order in ([0, 1, 2], [2, 1, 0], [1, 2, 0]):
        t, _, d = one_point(1, [cands[i] for i in order])
        assert t.tolist() == [2] and d.tolist() == [0.0]


def total_key(x):
    b = int(np.array([x], np.float32).view(np.uint32)[0])
    return (~b & 0xFFFFFFFF) if b & 0x80000000 else (b | 0x80000000)


def brute(num_points, l_max, records):
    """Each hash's best (dist total order, target, hash) candidate, then the
    l_max best of those, by ascending hash."""
    per = [dict() for _ in range(num_points)]
    for r in records:
        s, c, h, x = int(r["src"]), int(r["dst"]), int(r["hash"]), float(r["dist"])
        key = (total_key(x), c, h)
        cur = per[s].get(h)
        if cur is None or key < cur[0]:
            per[s][h] = (key, c, x)
    out = []
    for p in range(num_points):
        best = sorted(per[p].values(), key=lambda v: v[0])[:l_max]
        best.sort(key=lambda v: v[0][2])
        out.append([(v[1], v[0][2], v[2]) for v in best])
    return out


def random_stream(rng, num_points, n, hash_bits, dist_levels):
    src = rng.integers(0, num_points, n)
    dst = rng.integers(0, 4 * num_points, n)
    # a target's hash is a function of (src, dst), as compute_hash is for sketches
    hsh = ((src * 2654435761 + dst * 40503) >> 7) % (1 << hash_bits)
    dist = rng.integers(0, dist_levels, n).astype(np.float32) * np.float32(0.25)
    out = np.zeros(n, O.EDGE_DTYPE)
    out["src"] = src
    out["dst"] = dst
    out["hash"] = hsh
    out["dist"] = dist
    return out


@pytest.mark.parametrize("seed,num_points,n,l_max,hash_bits,levels", [
    (1, 5, 400, 4, 3, 7),       # heavy hash collisions and distance ties
    (2, 17, 2000, 8, 5, 50),
    (3, 3, 3000, 64, 12, 1000),  # default l_max and m_hash_bits
    (4, 40, 5000, 3, 2, 3),
])
def test_matches_brute_force(seed, num_points, n, l_max, hash_bits, levels):
    rng = np.random.default_rng(seed)
    r = random_stream(rng, num_points, n, hash_bits, levels)
    t, hs, d, cnt = O.hashprune_reduce(num_points, l_max, r)
    want = brute(num_points, l_max, r)
    for p in range(num_points):
        got = list(zip(t[p, :cnt[p]].tolist(), hs[p, :cnt[p]].tolist(), d[p, :cnt[p]].tolist()))
        assert got == want[p], p
        assert np.all(t[p, cnt[p]:] == 0xFFFFFFFF)


def test_invariant_under_shuffles_and_duplicates():
    rng = np.random.default_rng(7)
    r = random_stream(rng, 9, 1500, 4, 20)
    r = np.concatenate([r, r[:300]])  # an edge can arrive from several leaves
    base = O.hashprune_reduce(9, 6, r)
    for _ in range(5):
        perm = rng.permutation(len(r))
        got = O.hashprune_reduce(9, 6, r[perm])
        for a, b in zip(base, got):
            assert np.array_equal(a, b)


def test_slots_in_ascending_hash_and_capped():
    rng = np.random.default_rng(11)
    r = random_stream(rng, 4, 3000, 10, 500)
    t, hs, d, cnt = O.hashprune_reduce(4, 16, r)
    assert np.all(cnt == 16)
    for p in range(4):
        assert np.all(np.diff(hs[p].astype(np.int64)) > 0)


def test_empty_and_out_of_range():
    t, hs, d, cnt = O.hashprune_reduce(3, 4, np.zeros(0, O.EDGE_DTYPE))
    assert np.all(cnt == 0) and np.all(t == 0xFFFFFFFF)
    with pytest.raises(ValueError):
        O.hashprune_reduce(3, 4, recs([(0, 1, 1, 1.0), (3, 1, 1, 1.0)]))
