"""Pins the CPU oracle (oracle/) against the reference's known-answer tests,
closed forms, hand-worked cases and independent brute force (tests/brute.py).
"""
import math

import numpy as np
import pytest

import brute

F32 = np.float32


# ---- quantizer ----------------------------------------------------------------

def test_quantizer_reference_kat(orc):
    # dco_sq_int8.rs:3261-3283
    codes, scales, norms = orc.quantize(np.array([[0, 0, 0], [1, -1, 0.5]], np.float32), k_align=8)
    assert codes.shape == (2, 8)
    assert scales[0] == 1.0 and norms[0] == 0.0
    assert codes[0].tolist() == [0] * 8
    assert scales[1] == F32(1.0) / F32(127.0)
    assert norms[1] == 2.25
    assert codes[1].tolist() == [127, -127, 64, 0, 0, 0, 0, 0]


def test_quantizer_bits_kat(orc):
    # dco_sq_int8.rs:3285-3299
    c8, s8, _ = orc.quantize(np.array([[1, -1, 0.5]], np.float32), k_align=8, bits=8)
    assert s8[0] == F32(1.0) / F32(127.0)
    assert c8[0].tolist() == [127, -127, 64, 0, 0, 0, 0, 0]
    c4, s4, _ = orc.quantize(np.array([[1, -1, 0.5]], np.float32), k_align=8, bits=4)
    assert s4[0] == F32(1.0) / F32(7.0)
    assert c4[0, 0] == 7 and c4[0, 1] == -7
    assert np.all((c4 >= -7) & (c4 <= 7))


def test_quantizer_rounds_half_away_from_zero(orc):
    # max |x| = 127 gives scale exactly 1.0, so x/scale hits .5 exactly.
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5]], np.float32)
    codes, scales, _ = orc.quantize(x)
    assert scales[0] == 1.0
    assert codes[0, :7].tolist() == [127, 3, -3, 1, -1, 2, -127]


def test_quantizer_rejects_non_finite(orc):
    for bad in (np.nan, np.inf, -np.inf):
        x = np.ones((3, 5), np.float32)
        x[1, 2] = bad
        with pytest.raises(ValueError):
            orc.quantize(x)


def test_quantizer_padding_and_norm_are_sequential(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((40, 37)) * rng.uniform(0.01, 10, (40, 1))).astype(np.float32)
    codes, scales, norms = orc.quantize(x)
    assert codes.shape == (40, 48)
    assert np.all(codes[:, 37:] == 0)
    for r in range(40):
        c, s, n = brute.quantize_row(x[r])
        assert codes[r, :37].tolist() == c.tolist()
        assert scales[r].view(np.uint32) == np.float32(s).view(np.uint32)
        assert norms[r].view(np.uint32) == np.float32(n).view(np.uint32)


# ---- dots ---------------------------------------------------------------------

@pytest.mark.parametrize("n", [16, 32, 48, 64, 96, 128, 144, 768, 1024, 4096])
def test_dot_paths_match_int64(orc, n):
    rng = np.random.default_rng(n)
    a = rng.integers(-127, 128, n, dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, n, dtype=np.int64).astype(np.int8)
    ext_a = np.full(n, 127, np.int8)
    ext_b = np.full(n, -127, np.int8)
    best = orc.dot_kernel()
    try:
        for kernel in range(best + 1):
            orc.set_dot_kernel(kernel)
            for x, y in ((a, b), (ext_a, ext_b), (ext_a, ext_a), (a, a)):
                want = int(np.dot(x.astype(np.int64), y.astype(np.int64)))
                assert orc.dot(x, y) == want, (kernel, n)
                assert orc.dot(x, y, scalar=True) == want
    finally:
        orc.set_dot_kernel(best)


def test_dot_and_distance_reference_kat(orc):
    # dco_sq_int8.rs:3301-3325
    codes, scales, norms = orc.quantize(np.array([[1.0, 0.5], [0.5, 1.0]], np.float32), k_align=4)
    d = orc.dot(codes[0], codes[1])
    assert d == 127 * 64 + 64 * 127
    approx = orc.leaf_l2(d, scales[0], norms[0], scales[1], norms[1])
    expected = norms[0] + norms[1] - 2.0 * (F32(d) * scales[0] * scales[1])
    assert abs(float(approx) - float(expected)) < 1e-6


def test_leaf_distance_is_stepwise_f32(orc):
    rng = np.random.default_rng(7)
    for _ in range(2000):
        dot = int(rng.integers(-12_386_304, 12_386_305))
        rs, cs = rng.uniform(1e-4, 2e-2, 2).astype(np.float32)
        rn, cn = rng.uniform(0.1, 3.0, 2).astype(np.float32)
        got = orc.leaf_l2(dot, rs, rn, cs, cn)
        want = brute.leaf_dist(dot, rs, rn, cs, cn)
        assert got.view(np.uint32) == want.view(np.uint32)
        # and it is the f32 rounding of each step of the exact expression
        exact = (float(rn) + float(cn)) - 2.0 * (float(rs) * float(cs) * dot)
        assert math.isclose(max(exact, 0.0), float(got), rel_tol=1e-5, abs_tol=1e-6)


def test_distance_clamps_at_zero(orc):
    # identical vectors: n + n - 2*s*s*dot can round below zero; result is +0.0
    codes, scales, norms = orc.quantize(np.full((1, 64), 0.3, np.float32))
    d = orc.dot(codes[0], codes[0])
    v = orc.leaf_l2(d + 5, scales[0], norms[0], scales[0], norms[0])
    assert v == 0.0 and not np.signbit(v)
    w = orc.assign_l2(d + 5, scales[0], norms[0], scales[0], norms[0])
    assert w == 0.0 and not np.signbit(w)


def test_assign_distance_is_stepwise_f32(orc):
    rng = np.random.default_rng(8)
    for _ in range(2000):
        dot = int(rng.integers(-12_386_304, 12_386_305))
        ps, ls = rng.uniform(1e-4, 2e-2, 2).astype(np.float32)
        pn, ln = rng.uniform(0.1, 3.0, 2).astype(np.float32)
        got = orc.assign_l2(dot, ps, pn, ls, ln)
        want = brute.assign_dist(dot, ps, pn, ls, ln)
        assert got.view(np.uint32) == want.view(np.uint32)


# ---- row top-k ----------------------------------------------------------------

def test_rowtopk_without_ties_is_the_k_smallest_sorted(orc):
    rng = np.random.default_rng(11)
    for trial in range(50):
        n = int(rng.integers(1, 200))
        k = int(rng.integers(1, 33))
        # distances on a 1e-3 grid: all pairs differ by more than eps
        d = (rng.permutation(10_000)[:n] * 1e-3).astype(np.float32)
        ids = rng.permutation(1 << 20)[:n].astype(np.uint32)
        t = orc.RowTopK()
        for x, i in zip(d, ids):
            t.push(k, float(x), int(i))
        order = np.argsort(d, kind="stable")[: min(k, n)]
        assert [i for i, _ in t.items()] == ids[order].tolist()


def test_rowtopk_eps_tie_prefers_smaller_id(orc):
    t = orc.RowTopK()
    t.push(4, 0.5, 7)
    t.push(4, 0.50001, 3)  # within 2e-5: id 3 wins despite the larger distance
    t.push(4, 0.2, 9)
    assert [i for i, _ in t.items()] == [9, 3, 7]


def test_rowtopk_non_transitive_chain_depends_on_order(orc):
    # a~b and b~c are eps-ties, a and c are not: the answer depends on order.
    chain = [(0.0, 100), (1.5e-5, 99), (3.0e-5, 98)]
    t = orc.RowTopK()
    for d, i in chain:
        t.push(1, d, i)
    assert t.items() == [(98, pytest.approx(3.0e-5))]  # each newcomer wins its tie
    t = orc.RowTopK()
    for d, i in reversed(chain):
        t.push(1, d, i)
    assert t.items() == [(100, 0.0)]  # 99 loses the tie to 98, 100 is strictly closer


def test_rowtopk_matches_brute_force_with_many_ties(orc):
    rng = np.random.default_rng(12)
    for trial in range(200):
        n = int(rng.integers(1, 80))
        k = int(rng.integers(1, 33))
        d = (rng.integers(0, 12, n) * 1.1e-5).astype(np.float32)  # dense eps-chains
        ids = rng.integers(0, 50, n).astype(np.uint32)
        t = orc.RowTopK()
        for x, i in zip(d, ids):
            t.push(k, float(x), int(i))
        want = brute.rowtopk(k, [(F32(x), int(i)) for x, i in zip(d, ids)])
        got = t.items()
        assert [i for i, _ in got] == [i for _, i in want]
        assert [F32(x).view(np.uint32) for _, x in got] == [F32(x).view(np.uint32) for x, _ in want]


# ---- leaf operator --------------------------------------------------------------

def _random_sq8(orc, rows, dim, seed, dup_rows=()):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    for a, b in dup_rows:
        x[b] = x[a]
    return orc.quantize(x)


@pytest.mark.parametrize("n,k", [(2, 32), (3, 1), (17, 32), (33, 32), (40, 5), (64, 32)])
def test_leaf_topk_matches_brute_force(orc, n, k):
    codes, scales, norms = _random_sq8(orc, n + 5, 24, seed=n * 31 + k, dup_rows=[(1, 2)])
    gids = np.random.default_rng(n).permutation(10_000)[: n + 5].astype(np.uint32)
    members = np.random.default_rng(k).permutation(n + 5)[:n].astype(np.uint32)
    ids, d = orc.leaf_topk(codes, scales, norms, gids, members, [0], [n], k)
    bid, bd = brute.leaf_topk(codes, scales, norms, gids, members, k)
    assert ids.tolist() == bid.tolist()
    assert d.view(np.uint32).tolist() == bd.view(np.uint32).tolist()
    # invariants: never self, only members, k_eff slots filled
    keff = min(k, n - 1)
    mem_g = set(gids[members].tolist())
    for r in range(n):
        row = ids[r * k:(r + 1) * k]
        assert gids[members[r]] not in row.tolist()
        assert set(row[:keff].tolist()) <= mem_g
        assert np.all(row[keff:] == 0xFFFFFFFF)


def test_leaf_topk_multi_leaf_offsets(orc):
    codes, scales, norms = _random_sq8(orc, 300, 40, seed=3)
    gids = np.arange(300, dtype=np.uint32) * 3 + 1
    sizes = [70, 1, 2, 97, 130]
    members = np.random.default_rng(9).permutation(300).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    k = 8
    ids, d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, k)
    o = 0
    for off, n in zip(offs, sizes):
        bid, bd = brute.leaf_topk(codes, scales, norms, gids, members[off:off + n], k)
        assert ids[o:o + n * k].tolist() == bid.tolist()
        assert d[o:o + n * k].view(np.uint32).tolist() == bd.view(np.uint32).tolist()
        o += n * k


# ---- assignment ------------------------------------------------------------------

def test_hash64_is_splitmix64(orc):
    # SplitMix64 (Steele, Lea, Flood; Vigna's reference code) seeded with 0
    # emits these values; each is the finalizer applied to i*0x9e3779b97f4a7c15.
    gamma = 0x9E3779B97F4A7C15
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for i, w in enumerate(want, start=1):
        assert orc.hash64((i * gamma) & ((1 << 64) - 1)) == w
        assert brute.hash64((i * gamma) & ((1 << 64) - 1)) == w
    assert orc.assign_tie_key(5, 9) == brute.hash64((5 << 32) ^ 9 ^ gamma)


def _assign_case(orc, rows, dim, leaders, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    codes, scales, norms = orc.quantize(x)
    gids = rng.permutation(1 << 16)[:rows].astype(np.uint32)
    members = np.arange(rows, dtype=np.uint32)
    lead = rng.permutation(rows)[:leaders].astype(np.uint32)
    return codes, scales, norms, gids, members, lead


def test_assign_replay_matches_strict_order_without_near_ties(orc):
    codes, scales, norms, gids, members, lead = _assign_case(orc, 400, 64, 24, seed=21)
    args = (codes, scales, norms, gids, members, lead, [0], [400], [0], [24], [4])
    ids_a, d_a = orc.assign_replay(*args)
    ids_s, d_s = orc.assign_strict(*args)
    # find rows whose 5 best distances are pairwise more than eps apart
    ok_rows = 0
    for r in range(400):
        ds = np.sort(np.array([brute.assign_dist(orc.dot(codes[r], codes[l]), scales[r], norms[r], scales[l],
                                                 norms[l]) for l in lead], np.float32))
        if np.all(np.diff(ds[:5]) > 2e-5):
            ok_rows += 1
            assert ids_a[4 * r:4 * r + 4].tolist() == ids_s[4 * r:4 * r + 4].tolist()
            assert d_a[4 * r:4 * r + 4].view(np.uint32).tolist() == d_s[4 * r:4 * r + 4].view(np.uint32).tolist()
    assert ok_rows > 300


def test_assign_replay_tie_key_decides_exact_ties(orc):
    # two leaders with identical codes: distances are exactly equal, so the
    # SplitMix64 key of (member, leader) orders them (compute_backend.rs:6541-6553)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 32)).astype(np.float32)
    x[4] = x[5]
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(6, dtype=np.uint32) + 100
    for member in range(4):
        ids, _ = orc.assign_replay(codes, scales, norms, gids, [member], [4, 5], [0], [1], [0], [2], [2])
        k4, k5 = brute.hash64((member << 32) ^ 4 ^ 0x9E3779B97F4A7C15), brute.hash64(
            (member << 32) ^ 5 ^ 0x9E3779B97F4A7C15)
        first = 104 if k4 < k5 else 105
        assert ids[0] == first
        ids_rev, _ = orc.assign_replay(codes, scales, norms, gids, [member], [5, 4], [0], [1], [0], [2], [2])
        assert ids_rev[0] == first  # slot order does not matter for an exact tie
