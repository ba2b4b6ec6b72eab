"""GPU parity of the leaf operator (MFMA and exact executors) with the oracle,
through the C ABI.  Bar: ids and f32 distance bits identical."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_same, require_gpu, run_leaf, to_dev_sq8
from golden import make_golden as G
from shear_amd import _native as N
from shear_amd import datagen

pytestmark = pytest.mark.gpu

FIX = np.load(G.OUT)


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


@pytest.mark.parametrize("executor", [N.EXEC_MFMA, N.EXEC_EXACT])
@pytest.mark.parametrize("k", [2, 32])
def test_golden_formula_a(gpu, orc, executor, k):
    codes, scales, norms = orc.quantize(G.inputs_a())
    sq8 = to_dev_sq8(codes, scales, norms)
    ids, d, ctr = run_leaf(sq8, np.arange(607), np.arange(607), [0], [607], k, executor)
    assert_same(ids, d, FIX[f"a_leaf_k{k}_ids"], FIX[f"a_leaf_k{k}_dbits"].view(np.float32), f"A k={k}")
    assert ctr[N.C_LEAF_ROWS] == 607


@pytest.mark.parametrize("executor", [N.EXEC_MFMA, N.EXEC_EXACT])
@pytest.mark.parametrize("k", [2, 32])
def test_golden_formula_b_multi_leaf(gpu, orc, executor, k):
    codes, scales, norms = orc.quantize(G.inputs_b())
    sq8 = to_dev_sq8(codes, scales, norms)
    n = codes.shape[0]
    ids, d, _ = run_leaf(sq8, np.arange(n), np.arange(n), [0, 740, 1468], [740, 728, 641], k, executor)
    assert_same(ids, d, FIX[f"b_leaf_k{k}_ids"], FIX[f"b_leaf_k{k}_dbits"].view(np.float32), f"B k={k}")


@pytest.mark.parametrize("executor", [N.EXEC_MFMA, N.EXEC_EXACT])
def test_golden_formula_c_duplicates(gpu, executor):
    codes, scales, norms, gids = G.inputs_c()
    sq8 = to_dev_sq8(codes, scales, norms)
    ids, d, _ = run_leaf(sq8, gids, np.arange(20), [0], [20], 4, executor)
    assert_same(ids, d, FIX["c_leaf_k4_ids"], FIX["c_leaf_k4_dbits"].view(np.float32), "C")


def _gmm_case(orc, n, dim, seed, sigma=0.3, comps=8):
    x = datagen.gmm_numpy(n, dim, comps, sigma, seed)
    codes, scales, norms = orc.quantize(x)
    rng = np.random.default_rng(seed)
    gids = rng.permutation(1 << 24)[:n].astype(np.uint32)
    return codes, scales, norms, gids


@pytest.mark.parametrize("dim", [16, 100, 128, 768, 1000])
def test_random_leaves_match_oracle(gpu, orc, dim):
    sizes = [1, 2, 3, 31, 32, 33, 64, 127, 128, 129, 300, 1024]
    n = sum(sizes) + 17
    codes, scales, norms, gids = _gmm_case(orc, n, dim, seed=dim)
    members = np.random.default_rng(dim + 1).permutation(n)[: sum(sizes)].astype(np.uint32)  # gathered
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    sq8 = to_dev_sq8(codes, scales, norms, dim)
    for k in (1, 7, 32):
        want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, k)
        ids, d, ctr = run_leaf(sq8, gids, members, offs, sizes, k, N.EXEC_MFMA)
        assert_same(ids, d, want_ids, want_d, f"mfma dim={dim} k={k}")
        assert ctr[N.C_LEAF_ROWS] == sum(sizes)
    ids, d, _ = run_leaf(sq8, gids, members, offs, sizes, 32, N.EXEC_EXACT)
    assert_same(ids, d, want_ids, want_d, f"exact dim={dim}")


def test_empty_leaves_between_real_ones(gpu, orc):
    """Leaves without rows get no work items (the device-side item list
    skips them); the others, including ones of 1 and 1024 rows, match the
    oracle and every real row is counted once."""
    sizes = [0, 5, 0, 0, 300, 0, 1024, 0, 1, 0]
    n = sum(sizes) + 9
    codes, scales, norms, gids = _gmm_case(orc, n, 768, seed=5)
    members = np.random.default_rng(6).permutation(n)[: sum(sizes)].astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    sq8 = to_dev_sq8(codes, scales, norms, 768)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, 32)
    ids, d, ctr = run_leaf(sq8, gids, members, offs, sizes, 32, N.EXEC_MFMA)
    assert_same(ids, d, want_ids, want_d, "mfma with empty leaves")
    assert ctr[N.C_LEAF_ROWS] == sum(sizes)


def test_large_leaves_and_k_match_oracle(gpu, orc):
    sizes = [2048, 4096, 1500]
    n = sum(sizes)
    codes, scales, norms, gids = _gmm_case(orc, n, 96, seed=5, sigma=0.15, comps=3)
    members = np.arange(n, dtype=np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    sq8 = to_dev_sq8(codes, scales, norms, 96)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, 32)
    ids, d, _ = run_leaf(sq8, gids, members, offs, sizes, 32, N.EXEC_MFMA)
    assert_same(ids, d, want_ids, want_d, "large leaves")


def test_forced_exact_rerun_path_matches_oracle(gpu, orc):
    # The test knob sends every 4th / 20th row through the exact re-run kernel.
    sizes = [200, 513]
    n = sum(sizes)
    codes, scales, norms, gids = _gmm_case(orc, n, 64, seed=9)
    members = np.arange(n, dtype=np.uint32)
    offs = [0, 200]
    sq8 = to_dev_sq8(codes, scales, norms, 64)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, 32)
    for cap in (4, 20):
        ids, d, ctr = run_leaf(sq8, gids, members, offs, sizes, 32, N.EXEC_MFMA, debug_rerun_every=cap)
        assert_same(ids, d, want_ids, want_d, f"cap={cap}")
        assert ctr[N.C_LEAF_FALLBACK_ROWS] > 0
        assert ctr[N.C_LEAF_ROWS] == n


def test_forced_exact_rerun_leaves_longer_than_one_chunk(gpu, orc):
    # The re-run kernel computes a row's distances 1,024 columns at a time:
    # leaves of 2,500 (three chunks) and 1,100 rows, a one-row leaf, and a k
    # that leaves output rows unaligned to 16 bytes.
    sizes = [2500, 1, 1100]
    n = sum(sizes)
    codes, scales, norms, gids = _gmm_case(orc, n, 96, seed=11, sigma=0.2, comps=4)
    members = np.arange(n, dtype=np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    sq8 = to_dev_sq8(codes, scales, norms, 96)
    for k in (32, 13):
        want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, k)
        ids, d, ctr = run_leaf(sq8, gids, members, offs, sizes, k, N.EXEC_MFMA, debug_rerun_every=3)
        assert_same(ids, d, want_ids, want_d, f"k={k}")
        assert ctr[N.C_LEAF_FALLBACK_ROWS] > 0
        assert ctr[N.C_LEAF_ROWS] == n


def test_heavy_tie_data_matches_oracle(gpu, orc):
    # few distinct code patterns -> exact and eps ties everywhere
    rng = np.random.default_rng(3)
    base = rng.integers(-3, 4, (6, 48)).astype(np.float32)
    x = base[rng.integers(0, 6, 700)] + rng.integers(0, 2, (700, 48)) * 0.01
    codes, scales, norms = orc.quantize(x.astype(np.float32))
    gids = rng.permutation(5000)[:700].astype(np.uint32)
    members = np.arange(700, dtype=np.uint32)
    sq8 = to_dev_sq8(codes, scales, norms, 48)
    for k in (3, 32):
        want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, [0], [700], k)
        ids, d, _ = run_leaf(sq8, gids, members, [0], [700], k, N.EXEC_MFMA)
        assert_same(ids, d, want_ids, want_d, f"ties k={k}")


def test_mfma_is_deterministic(gpu, orc):
    codes, scales, norms, gids = _gmm_case(orc, 4096, 128, seed=2)
    sq8 = to_dev_sq8(codes, scales, norms, 128)
    sizes = [1024] * 4
    offs = [0, 1024, 2048, 3072]
    a = run_leaf(sq8, gids, np.arange(4096), offs, sizes, 32, N.EXEC_MFMA)
    b = run_leaf(sq8, gids, np.arange(4096), offs, sizes, 32, N.EXEC_MFMA)
    assert_same(a[0], a[1], b[0], b[1], "repeat")


def test_c2_shaped_leaves_match_oracle(gpu, orc):
    # The leaf-microbench shape (1024 x 768 SQ8 leaves from a unit-norm GMM)
    # on a few leaves, checked against the oracle bit for bit.
    leaves = 6
    x = datagen.gmm_numpy(leaves * 1024, 768, leaves, 0.3, seed=1)
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(leaves * 1024, dtype=np.uint32)
    members = np.arange(leaves * 1024, dtype=np.uint32)
    offs = np.arange(leaves) * 1024
    sizes = [1024] * leaves
    sq8 = to_dev_sq8(codes, scales, norms, 768)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, 32)
    ids, d, ctr = run_leaf(sq8, gids, members, offs, sizes, 32, N.EXEC_MFMA)
    assert_same(ids, d, want_ids, want_d, "C2-shaped")
    # the exact re-run is the exception, not the rule, on realistic data
    assert ctr[N.C_LEAF_FALLBACK_ROWS] < 0.05 * leaves * 1024


_FRESH = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
from gpu_helpers import run_leaf, to_dev_sq8
from oracle import pyoracle as orc
from shear_amd import _native as N
rng = np.random.default_rng(5)
codes, scales, norms = orc.quantize(rng.standard_normal((40, 32)).astype(np.float32))
ids, d, _ = run_leaf(to_dev_sq8(codes, scales, norms), np.arange(40), np.arange(40), [0], [40], 8, N.EXEC_MFMA)
want_ids, want_d = orc.leaf_topk(codes, scales, norms, np.arange(40, dtype=np.uint32),
                                 np.arange(40, dtype=np.uint32), np.array([0]), [40], 8)
assert np.array_equal(ids, want_ids) and np.array_equal(d.view(np.uint32), want_d.view(np.uint32))
print("fresh-process leaf ok", flush=True)
"""


def test_tiny_batch_in_a_fresh_process(gpu):
    # The per-device leaf workspace grows and is kept, so in one process a
    # tiny batch after a large one never sees a tiny workspace.  A fresh
    # process runs the tiny case first (regression: the persistent grid had
    # no workgroup when the survivor log held fewer than 16 slots).
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "fresh-process leaf ok" in r.stdout
