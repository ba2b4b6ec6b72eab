"""CPU oracle of HashPrune with a named R-half backfill policy
(orc_hashprune_rhalf_reduce: SoftTier-Q3 and its siblings), pinned.

The `build_shear_index` binary builds with SoftTier-Q3, a row cap of 3 and
priority alpha 1.02 unless told otherwise (apps/build_shear_index/src/
main.rs:2360-2374, :3210); BASELINE's "HashPrune cap 3".

Pins (paths relative to shear-core/src/algorithm/pipnn/):
  * the reference's KAT hash_prune.rs:2699-2714 (the a2-versus-b1 boundary of
    the SoftTier priority at the default alpha) and the primary-prefix KAT
    :2505-2527 with its shortlist worked by hand;
  * full and empty rows get no shortlist (:2616-2621), a row cap cuts it
    (:2791-2828 shape);
  * an independent restatement below (dictionaries instead of sorted runs)
    of the reference's characterization :2601-2682 on random streams with
    heavy hash collisions, repeated targets and distance ties;
  * invariance under shuffles of the record stream, which the reference
    asserts for its streaming insert (:3019-3049, :3243-3290).
"""
import numpy as np
import pytest

from oracle import pyoracle as O
from test_hashprune_oracle import random_stream, total_key


def recs(cands, src=0):
    out = np.zeros(len(cands), O.EDGE_DTYPE)
    for i, (t, h, d) in enumerate(cands):
        out[i] = (src, t, h, 0, d)
    return out


def row(cands, l_max, **kw):
    t, hs, d, cnt, pc = O.hashprune_rhalf_reduce(1, l_max, recs(cands), **kw)
    return t[0, :cnt[0]].tolist(), int(pc[0])


def cross_layer_backups(a2):
    # hash_prune.rs:2468-2487 named_rhalf_cross_layer_backups, l_max 4, default alpha
    c = [(10, 10, 0.25), (101, 10, 0.30), (102, 10, a2), (20, 20, 0.25), (201, 20, 1.00)]
    r, _ = row(c, 4)
    return sorted(x for x in r if x >= 100)


def test_kat_soft_tier_a2_b1_boundary():
    assert cross_layer_backups(float(np.float32(0.90) * np.float32(0.90))) == [101, 102]
    assert cross_layer_backups(float(np.float32(0.95) * np.float32(0.95))) == [101, 201]


def test_kat_primary_prefix_and_hand_worked_shortlist():
    # hash_prune.rs:2505-2527: three primaries; the shortlist worked by hand:
    # groups h1 = [11 (1.1, layer 1), 12 (1.2, layer 2)], h2 = [21 (1.0, layer 1)];
    # capacity min(8 / 2, 8 - 3) = 4; SoftTier scores 21: 1.0, 11: 1.1, 12: 1.2 * 1.21
    c = [(10, 1, 1.0), (11, 1, 1.1), (12, 1, 1.2), (20, 2, 0.8), (21, 2, 1.0), (30, 3, 0.7)]
    r, pc = row(c, 8)
    assert pc == 3
    assert r == [10, 20, 30, 21, 11, 12]
    # distance-first ranks by distance only; hard-tier by layer first
    assert row(c, 8, mode="rhalf-distance-first-q3")[0] == [10, 20, 30, 21, 11, 12]
    c2 = [(10, 1, 1.0), (11, 1, 1.05), (12, 1, 1.06), (20, 2, 0.8), (21, 2, 1.2), (30, 3, 0.7)]
    assert row(c2, 8, mode="rhalf-hard-tier-q3")[0] == [10, 20, 30, 11, 21, 12]
    assert row(c2, 8, mode="rhalf-distance-first-q3")[0] == [10, 20, 30, 11, 12, 21]
    # hash-slot-1: quota 1, only each group's best
    assert row(c2, 8, mode="rhalf-hash-slot-1")[0] == [10, 20, 30, 11, 21]


def test_production_alpha_and_row_cap():
    # alpha 1.02: a layer-2 member at 1.0 (score 1.0404) beats a layer-1 at 1.05
    c = [(10, 1, 0.5), (11, 1, 0.9), (12, 1, 1.0), (20, 2, 0.5), (21, 2, 1.05), (30, 3, 0.5), (31, 3, 1.5)]
    r, pc = row(c, 8, priority_alpha=1.02)
    assert pc == 3 and r[3:] == [11, 12, 21, 31]
    r, _ = row(c, 8, priority_alpha=1.1)  # 1.0 * 1.21 > 1.05
    assert r[3:] == [11, 21, 12, 31]
    r, _ = row(c, 8, priority_alpha=1.02, row_cap=3)
    assert r[3:] == [11, 12, 21]
    # the capacity never exceeds the spare slots: 3 primaries, l_max 4
    r, _ = row(c, 4, priority_alpha=1.02, row_cap=3)
    assert r == [10, 20, 30, 11]


def test_full_and_empty_rows_get_no_shortlist():
    c = [(1000 + h * 10 + k, h, 1.0 + 0.01 * k + 0.001 * h) for h in range(8) for k in range(4)]
    r, pc = row(c, 8, row_cap=3)
    assert pc == 8 and len(r) == 8
    t, hs, d, cnt, pc = O.hashprune_rhalf_reduce(3, 8, recs(c, src=1))
    assert cnt.tolist() == [0, 8, 0] and pc.tolist() == [0, 8, 0]


def test_primary_target_and_repeats_are_not_backups():
    # the primary's own target at a worse distance, and a target repeated at
    # several distances (kept at its best) in the group
    c = [(10, 1, 0.5), (10, 1, 0.9), (11, 1, 1.2), (11, 1, 0.7), (12, 1, 0.8)]
    assert row(c, 8)[0] == [10, 11, 12]


def brute_rhalf(num_points, l_max, records, quota, row_cap, alpha_sq, mode):
    """The reference characterization hash_prune.rs:2601-2682, restated with
    dictionaries."""
    per = [dict() for _ in range(num_points)]  # hash -> {target: (key, dist)}
    for r in records:
        s, c, h, x = int(r["src"]), int(r["dst"]), int(r["hash"]), float(r["dist"])
        key = (total_key(x), c, h)
        g = per[s].setdefault(h, {})
        if c not in g or key < g[c][0]:
            g[c] = (key, x)
    out = []
    for p in range(num_points):
        best = {h: min(g.values(), key=lambda v: v[0]) for h, g in per[p].items()}
        prim = sorted(best.items(), key=lambda kv: kv[1][0])[:l_max]
        prim.sort(key=lambda kv: kv[0])
        rowl = [(v[0][1], h, v[1]) for h, v in prim]
        if 0 < len(prim) < l_max:
            members = []
            for h, v in prim:
                others = sorted((val for t, val in per[p][h].items() if t != v[0][1]), key=lambda q: q[0])[:quota]
                for layer, (key, x) in enumerate(others, 1):
                    members.append((key, x, layer))

            def prio(m):
                key, x, layer = m
                if mode == "rhalf-soft-tier-q3":
                    sc = float(np.float64(x) * (alpha_sq ** (layer - 1))) if layer < 3 else \
                        float(np.float64(x) * alpha_sq * alpha_sq)
                    return (sc, layer, key[1], key[2])
                if mode == "rhalf-hard-tier-q3":
                    return (layer, key)
                return (key[0], layer, key[1], key[2])

            members.sort(key=prio)
            budget = l_max // 2
            cap = row_cap if row_cap and row_cap < budget else budget
            for key, x, layer in members[:min(cap, l_max - len(prim))]:
                rowl.append((key[1], key[2], x))
        out.append(rowl)
    return out


@pytest.mark.parametrize("mode", ["rhalf-soft-tier-q3", "rhalf-distance-first-q3", "rhalf-hard-tier-q3",
                                  "rhalf-hash-slot-1"])
@pytest.mark.parametrize("seed,num_points,n,l_max,hash_bits,levels,row_cap", [
    (1, 6, 500, 8, 3, 7, 0),       # heavy collisions and ties; rows near full
    (2, 20, 1500, 16, 4, 50, 3),   # underfull rows with many groups, cap 3
    (3, 4, 3000, 64, 4, 1000, 3),  # default R, production cap, groups of colliding targets
    (4, 30, 800, 5, 2, 3, 2),      # odd l_max
])
def test_matches_independent_restatement(mode, seed, num_points, n, l_max, hash_bits, levels, row_cap):
    rng = np.random.default_rng(seed)
    r = random_stream(rng, num_points, n, hash_bits, levels)
    if seed == 2:  # repeated targets at other distances
        extra = r[rng.integers(0, n, n // 4)].copy()
        extra["dist"] = rng.integers(0, levels, len(extra)).astype(np.float32) * np.float32(0.25)
        r = np.concatenate([r, extra])
    quota = 1 if mode == "rhalf-hash-slot-1" else 3
    alpha = 1.02
    t, hs, d, cnt, pc = O.hashprune_rhalf_reduce(num_points, l_max, r, mode=mode, row_cap=row_cap,
                                                 priority_alpha=alpha)
    want = brute_rhalf(num_points, l_max, r, quota, row_cap, float(np.float64(np.float32(alpha)) ** 2), mode)
    backfilled = 0
    for p in range(num_points):
        got = list(zip(t[p, :cnt[p]].tolist(), hs[p, :cnt[p]].tolist(), d[p, :cnt[p]].tolist()))
        assert got == want[p], (p, got, want[p])
        backfilled += int(cnt[p] - pc[p])
    if seed in (2, 3):
        assert backfilled > 0  # the case exercises the shortlist


def test_invariant_under_shuffles():
    rng = np.random.default_rng(9)
    r = random_stream(rng, 12, 2000, 5, 40)
    base = O.hashprune_rhalf_reduce(12, 16, r, row_cap=3, priority_alpha=1.02)
    for _ in range(4):
        s = r[rng.permutation(len(r))]
        got = O.hashprune_rhalf_reduce(12, 16, s, row_cap=3, priority_alpha=1.02)
        for a, b in zip(base, got):
            assert np.array_equal(a, b)
