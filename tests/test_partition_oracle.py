"""Pins the subtree partition restatement (oracle/tessa_partition.c) with the
reference's known-answer tests, closed forms, hand-built known partitions,
structural invariants and the independent Python restatement in brute.py."""
import numpy as np
import pytest

import brute
from shear_amd import datagen

F32 = np.float32


# ---- helpers the split control uses ----------------------------------------------

def test_adaptive_psamp_reference_kats(orc):
    # params.rs:4002-4020 (the f64 CPU twin of compute_backend.rs:7044-7075)
    assert orc.adaptive_psamp(0.001, 10_000, 0) == F32(0.001)
    assert orc.adaptive_psamp(0.001, 10_000_000, 0) == F32(F32(0.001) * F32(0.1))
    # 0.00005 in f64; in f32 the product lands one ulp above the clamp
    got = orc.adaptive_psamp(0.001, 10_000_000, 3)
    assert got == F32(F32(F32(0.001) * F32(0.1)) * F32(0.5)) and abs(float(got) - 5e-5) < 4e-12
    assert orc.adaptive_psamp(0.5, 1_000, 0) == F32(0.1)
    assert orc.adaptive_psamp(0.000001, 1_000, 0) == F32(0.00005)


@pytest.mark.parametrize("n,depth", [(99_999, 0), (100_000, 1), (1_000_000, 3), (5_000_000, 5),
                                      (20_000_000, 2), (12_345, 7)])
def test_adaptive_psamp_matches_brute(orc, n, depth):
    assert orc.adaptive_psamp(0.02, n, depth) == brute.adaptive_psamp(0.02, n, depth)


def test_meaningful_split_closed_form(orc):
    assert orc.meaningful_split(200, 199, 256)          # parent within the terminal limit
    assert orc.meaningful_split(5000, 256, 256)         # every child is a leaf
    assert not orc.meaningful_split(5000, 5000, 256)    # nothing shrank
    # min shrink = max(parent >> 5, 32): 10000 -> 312, 1000 -> 32
    assert orc.meaningful_split(10_000, 10_000 - 312, 256)
    assert not orc.meaningful_split(10_000, 10_000 - 311, 256)
    assert orc.meaningful_split(1000, 968, 256)
    assert not orc.meaningful_split(1000, 969, 256)
    for parent, child, term in [(10_000, 9_700, 256), (300, 290, 1), (2, 1, 0), (40, 39, 1)]:
        assert orc.meaningful_split(parent, child, term) == brute.meaningful(parent, child, term)


def test_sort_unique(orc):
    rng = np.random.default_rng(0)
    v = rng.integers(0, 50, 200)
    assert orc.sort_unique(v).tolist() == np.unique(v).tolist()
    assert orc.sort_unique([]).tolist() == []


def test_retry_leaders_take_one_row_per_span(orc):
    rows = np.arange(1000, 1997, dtype=np.uint32)  # 997 rows
    for nl, attempt in [(2, 1), (7, 2), (128, 3)]:
        got = orc.sample_retry_leaders(rows, nl, 0xABCDEF, attempt)
        for s in range(nl):
            b, e = s * 997 // nl, (s + 1) * 997 // nl
            e = max(e, b + 1)
            key = brute.hash64(0xABCDEF ^ ((attempt * 0xD6E8FEB86659FD93) & brute.M64)
                               ^ ((s * 0x9E3779B97F4A7C15) & brute.M64))
            assert got[s] == rows[b + key % (e - b)]
            assert rows[b] <= got[s] < rows[b] + (e - b)


def test_hash_ranked_leaders_are_the_smallest_keys(orc):
    pts = np.arange(0, 900, 3, dtype=np.uint32)
    for nl, attempt, depth in [(2, 0, 0), (16, 3, 2), (128, 5, 9)]:
        got = orc.hash_rank_leaders(pts, nl, 99, attempt, depth)
        keys = sorted((brute.hash64((99 ^ ((attempt * 0xBF58476D1CE4E5B9) & brute.M64) ^ (depth << 19)
                                     ^ (i << 7) ^ ((int(p) << 31) & brute.M64)) & brute.M64), int(p))
                      for i, p in enumerate(pts))
        assert got.tolist() == [p for _, p in keys[:nl]]


def test_root_seed_closed_form(orc):
    def rotl(x, r):
        return ((x << r) | (x >> (64 - r))) & brute.M64

    want = 42 ^ ((3 * 0x9E3779B97F4A7C15) & brute.M64) ^ rotl(1000, 17) ^ rotl(5000, 7) ^ rotl(64, 29)
    assert orc.subtree_root_seed(42, 3, 1000, 5000, 64) == want


def test_assign_before_tie_rule(orc):
    # outside 2e-5 the smaller distance wins; inside, the smaller SplitMix64 key
    assert orc.assign_before(1.0, 5, 9, 1.1, 3)
    assert not orc.assign_before(1.1, 5, 9, 1.0, 3)
    a, b = brute.tie_key(5, 9), brute.tie_key(5, 3)
    assert orc.assign_before(1.0, 5, 9, 1.00001, 3) == (a < b)
    assert orc.assign_before(1.00001, 5, 3, 1.0, 9) == (b < a)


# ---- whole partitions ----------------------------------------------------------------

def _gmm(n, dim, comps, seed, sigma=0.3):
    return datagen.gmm_numpy(n, dim, comps, sigma, seed)


CASES = [
    # n, dim, comps, fanout, leaf_max, psamp, leaf_min, root leaders
    (1500, 32, 6, 2, 256, 0.01, 64, None),
    (1200, 48, 6, 1, 100, 0.005, 64, None),   # retries
    (600, 16, 6, 3, 128, 0.02, 64, None),
    (300, 24, 6, 2, 512, 0.05, 64, None),     # small root (process_node)
    (700, 20, 5, 2, 1024, 0.05, 100, None),   # small root, merged small children
    (900, 32, 4, 2, 200, 0.01, 64, [5, 400, 800]),  # root leaders
    (2000, 64, 12, 4, 300, 0.004, 64, None),
]


@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}f{c[3]}m{c[4]}" for c in CASES])
def test_partition_matches_independent_restatement(orc, case):
    n, dim, comps, fan, lmax, ps, lmin, roots = case
    codes, scales, norms = orc.quantize(_gmm(n, dim, comps, n + dim))
    seed = 1234567 + n
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=seed, fanout_second=fan, leaf_max=lmax,
                                        leaf_min=lmin, psamp_fraction=ps, root_leaders=roots)
    want, flags = brute.partition(codes, scales, norms, seed=seed, fanout_second=fan, leaf_max=lmax,
                                  leaf_min=lmin, psamp=ps, root_leaders=roots)
    assert flags == 0 and ctr[7] == 0
    assert [list(x) for x in leaves] == [list(x) for x in want]


@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}f{c[3]}m{c[4]}" for c in CASES])
def test_partition_invariants(orc, case):
    n, dim, comps, fan, lmax, ps, lmin, roots = case
    codes, scales, norms = orc.quantize(_gmm(n, dim, comps, n + dim))
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=77, fanout_second=fan, leaf_max=lmax,
                                        leaf_min=lmin, psamp_fraction=ps, root_leaders=roots)
    sizes = [len(x) for x in leaves]
    assert all(0 < s <= lmax for s in sizes)
    for x in leaves:
        assert np.all(np.diff(x.astype(np.int64)) > 0)  # ascending, no repeats
    counts = np.bincount(np.concatenate(leaves), minlength=n)
    # every row reaches the leaves; replication only happens at the root
    assert counts.min() >= 1 and counts.max() <= fan
    assert ctr[13] == len(leaves) == ctr[36]            # OUTPUT_LEAF_COUNT, LEAF_SIZE_COUNT
    assert ctr[12] == sum(sizes) == ctr[35]             # OUTPUT_ROWS, LEAF_SIZE_SUM
    assert ctr[33] == min(sizes) and ctr[34] == max(sizes)
    assert ctr[21] == n


def test_well_separated_blocks_split_exactly(orc):
    # 4 tight clusters far apart, rows grouped by cluster: the ordinal leaders
    # (rows 0, 300, 600, 900) land one per cluster, so each cluster is a leaf.
    rng = np.random.default_rng(1)
    centres = np.eye(4, 24, dtype=np.float32) * 8.0
    x = np.concatenate([c + 0.01 * rng.standard_normal((300, 24)).astype(np.float32) for c in centres])
    codes, scales, norms = orc.quantize(x)
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=5, fanout_second=1, leaf_max=400,
                                        psamp_fraction=4 / 1200)
    assert [x.tolist() for x in leaves] == [list(range(i * 300, (i + 1) * 300)) for i in range(4)]
    assert ctr[130] == 0 and ctr[131] == 0


def test_balanced_fallback_is_even_odd(orc):
    # Root leaders (no retry allowed) whose split shrinks nothing: one leader in
    # the cluster, one far outlier.  The node falls back to even/odd rows.
    rng = np.random.default_rng(2)
    x = 0.01 * rng.standard_normal((400, 16)).astype(np.float32)
    x[399] = 10.0
    codes, scales, norms = orc.quantize(x)
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=9, fanout_second=1, leaf_max=256,
                                        root_leaders=[0, 399])
    assert [x.tolist() for x in leaves] == [list(range(0, 400, 2)), list(range(1, 400, 2))]
    assert ctr[131] == 1 and ctr[130] == 0


def test_depth_limit_raises_oversized_terminal_node(orc):
    codes, scales, norms = orc.quantize(_gmm(1500, 16, 4, 3))
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=1, fanout_second=1, leaf_max=100,
                                        psamp_fraction=0.002, max_depth=1)
    assert leaves is None and int(ctr[7]) & (1 << 10)


def test_leaf_capacity_raises_leaf_desc(orc):
    codes, scales, norms = orc.quantize(_gmm(1500, 16, 4, 3))
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=1, fanout_second=1, leaf_max=100,
                                        psamp_fraction=0.01, max_leaf_count=3)
    assert leaves is None and int(ctr[7]) & (1 << 2)
