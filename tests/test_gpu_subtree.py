"""GPU parity of the resident-subtree operator (recursive partition + leaf
top-k, tessa_session_run_subtree) with the CPU oracle.

Bar: leaf layout (leaf order, member order), the partition counters and the
top-k ids / f32 distance bits identical to the oracle's."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_same, require_gpu
from shear_amd import _native as N
from shear_amd import datagen
from shear_amd import subtree as S

pytestmark = pytest.mark.gpu

# the leaf operator's tile count and the walk's phase clocks (timings) have no
# oracle counterpart
SKIP_WORDS = {N.P_LEAF_SQ8_WMMA_TILES, *N.P_CLOCK_WORDS}


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _data(orc, n, dim, comps, seed, sigma=0.3):
    x = datagen.gmm_numpy(n, dim, comps, sigma, seed)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(seed).permutation(1 << 22)[:n].astype(np.uint32)
    return codes, scales, norms, gids


def _run(orc, codes, scales, norms, gids, dim, *, fan, leaf_max, psamp, k=32, leaf_min=64, roots=None,
         max_depth=10, max_leaders=128, depth=0, executor=N.EXEC_MFMA, partition_only=False, check_topk=True):
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    params = S.PiPNNSubtreeParams(leaf_knn=k, c_max=leaf_max, psamp_fraction=psamp, max_leaders=max_leaders,
                                  max_depth=max_depth, fanout_second=fan, random_seed=7, executor=executor,
                                  c_min=leaf_min)
    req = S.GpuSubtreePartitionRequest(point_ids=gids, root_leader_ids=roots, depth=depth,
                                       parent_points=len(gids) * 3, min_recurse_size=leaf_min)
    out = sess.run(req, params, partition_only=partition_only)
    torch.cuda.synchronize()
    seed = S.subtree_root_seed(7, depth, len(gids), len(gids) * 3, leaf_min)
    assert seed == orc.subtree_root_seed(7, depth, len(gids), len(gids) * 3, leaf_min)
    plan = S.plan_subtree(len(gids), k, min(max_leaders, 128), fan, None, leaf_max)
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=seed, root_depth=depth, max_depth=max_depth,
                                        max_leaders=min(max_leaders, 128), fanout_second=fan,
                                        leaf_min=plan.leaf_min, leaf_max=plan.leaf_max,
                                        psamp_fraction=psamp, root_leaders=roots,
                                        max_leaf_count=plan.max_leaf_count, max_leaf_rows=plan.max_leaf_rows)
    return sess, out, leaves, ctr, plan


def _check_layout(out, leaves, ctr):
    assert ctr[N.P_OVERFLOW_FLAGS] == 0
    assert out.leaf_count == len(leaves)
    lr = out.leaf_rows
    rows = out.leaf_row_ids[:lr].cpu().numpy().view(np.uint32)
    starts = out.leaf_starts[: out.leaf_count].cpu().numpy()
    sizes = out.leaf_sizes[: out.leaf_count].cpu().numpy()
    want_sizes = np.array([len(x) for x in leaves], np.int64)
    assert np.array_equal(sizes, want_sizes), "leaf sizes / order differ"
    assert np.array_equal(starts, np.concatenate([[0], np.cumsum(want_sizes)[:-1]]))
    assert np.array_equal(rows, np.concatenate(leaves)), "leaf member rows differ"
    for w in range(N.SUBTREE_COUNTER_WORDS):
        if w not in SKIP_WORDS:
            assert out.counters[w] == ctr[w], f"counter word {w}: gpu {out.counters[w]} oracle {ctr[w]}"


def _check_topk(orc, out, leaves, codes, scales, norms, gids):
    members = np.concatenate(leaves).astype(np.uint32)
    sizes = [len(x) for x in leaves]
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, out.k)
    n = out.leaf_rows * out.k
    ids = out.topk_ids[:n].cpu().numpy().view(np.uint32)
    d = out.topk_dists[:n].cpu().numpy()
    assert_same(ids, d, want_ids, want_d, "subtree top-k")


CASES = [
    # n, dim, comps, fanout, leaf_max, psamp, roots
    (1500, 32, 6, 2, 256, 0.01, None),
    (1200, 48, 6, 1, 100, 0.005, None),          # split retries
    (600, 16, 6, 3, 128, 0.02, None),
    (300, 24, 6, 2, 512, 0.05, None),            # small root: process_node path
    (900, 32, 4, 2, 256, 0.01, [5, 400, 800]),   # root leaders
    (2000, 64, 12, 4, 300, 0.004, None),
    (6000, 768, 16, 2, 1024, 0.002, None),       # C3 dims, multi-level
]


@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}d{c[1]}f{c[3]}" for c in CASES])
def test_subtree_matches_oracle(gpu, orc, case):
    n, dim, comps, fan, lmax, ps, roots = case
    codes, scales, norms, gids = _data(orc, n, dim, comps, n + dim)
    _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, dim, fan=fan, leaf_max=lmax, psamp=ps,
                                  roots=roots)
    _check_layout(out, leaves, ctr)
    _check_topk(orc, out, leaves, codes, scales, norms, gids)


@pytest.mark.parametrize("fan", [1, 2, 3, 4])
def test_subtree_near_tied_distances_match_oracle(gpu, orc, fan):
    """Rows on a 3-level grid, many of them repeated, each scaled by 1 + a
    few ulps: a row's distances to the leaders fall into a handful of values
    that differ by less than the tie band, so assignment turns on the hash
    tie key and the first-tile visit rule mostly meets a distance inside the
    band above its threshold (and must visit every leader)."""
    rng = np.random.default_rng(50 + fan)
    base = rng.integers(0, 3, (700, 16)).astype(np.float32)
    x = base[rng.integers(0, 700, 5000)]
    x *= (1.0 + rng.integers(0, 8, (5000, 1)) * 1e-7).astype(np.float32)
    codes, scales, norms = orc.quantize(x.astype(np.float32))
    gids = rng.permutation(1 << 22)[:5000].astype(np.uint32)
    _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 16, fan=fan, leaf_max=256, psamp=0.01, leaf_min=32)
    _check_layout(out, leaves, ctr)
    _check_topk(orc, out, leaves, codes, scales, norms, gids)


def test_subtree_unnormalised_rows_are_certified(gpu, orc):
    """C1-shaped rows (128-d, centres N(0, I), sigma 0.3, not normalised):
    their norms differ by far more than 1 %, so the filter tests each column
    against its own norm.  With the leaf-wide smallest norm the test let
    through so many candidates that about a third of the rows overflowed
    their logs and took the exact re-run; the rows must now be certified (a
    handful of re-runs at most) and still match the oracle bit for bit."""
    x = datagen.gmm_numpy(12000, 128, 64, 0.3, 0, unit_norm=False)
    codes, scales, norms = orc.quantize(x)
    assert (norms.max() - norms.min()) > 0.05 * norms.max()
    gids = np.arange(12000, dtype=np.uint32)
    _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 128, fan=2, leaf_max=1024, psamp=0.01)
    _check_layout(out, leaves, ctr)
    reruns = int(out.leaf_counters[N.C_LEAF_FALLBACK_ROWS])
    assert reruns <= out.leaf_rows // 100, f"{reruns} of {out.leaf_rows} rows re-run exactly"
    _check_topk(orc, out, leaves, codes, scales, norms, gids)


def test_subtree_exact_executor_and_small_k(gpu, orc):
    codes, scales, norms, gids = _data(orc, 2500, 40, 8, 11)
    for executor, k in [(N.EXEC_EXACT, 32), (N.EXEC_MFMA, 5)]:
        _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 40, fan=2, leaf_max=256, psamp=0.01, k=k,
                                      executor=executor)
        _check_layout(out, leaves, ctr)
        _check_topk(orc, out, leaves, codes, scales, norms, gids)


def test_subtree_balanced_fallback(gpu, orc):
    rng = np.random.default_rng(2)
    x = 0.01 * rng.standard_normal((400, 16)).astype(np.float32)
    x[399] = 10.0
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(400, dtype=np.uint32)
    _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 16, fan=1, leaf_max=256, psamp=0.01,
                                  roots=[0, 399])
    _check_layout(out, leaves, ctr)
    assert out.counters[N.P_LARGE_BALANCED_FALLBACKS] == 1
    _check_topk(orc, out, leaves, codes, scales, norms, gids)


def test_subtree_partition_only(gpu, orc):
    codes, scales, norms, gids = _data(orc, 3000, 24, 6, 21)
    _, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 24, fan=2, leaf_max=200, psamp=0.01,
                                  partition_only=True)
    _check_layout(out, leaves, ctr)
    assert out.k == 0


def test_subtree_repeat_is_deterministic(gpu, orc):
    codes, scales, norms, gids = _data(orc, 5000, 96, 10, 31)
    sess, out, leaves, ctr, _ = _run(orc, codes, scales, norms, gids, 96, fan=2, leaf_max=512, psamp=0.005)
    a = (out.leaf_row_ids[: out.leaf_rows].cpu(), out.topk_ids[: out.leaf_rows * out.k].cpu())
    params = S.PiPNNSubtreeParams(leaf_knn=32, c_max=512, psamp_fraction=0.005, max_leaders=128, fanout_second=2,
                                  random_seed=7, c_min=64)
    req = S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=len(gids) * 3, min_recurse_size=64)
    out2 = sess.run(req, params)
    torch.cuda.synchronize()
    assert torch.equal(a[0], out2.leaf_row_ids[: out2.leaf_rows].cpu())
    assert torch.equal(a[1], out2.topk_ids[: out2.leaf_rows * out2.k].cpu())


def test_subtree_depth_overflow_is_reported(gpu, orc):
    codes, scales, norms, gids = _data(orc, 1500, 16, 4, 3)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, 16)
    params = S.PiPNNSubtreeParams(leaf_knn=8, c_max=100, psamp_fraction=0.002, max_leaders=128, max_depth=1,
                                  fanout_second=1)
    with pytest.raises(N.TessaError) as ei:
        sess.run(S.GpuSubtreePartitionRequest(point_ids=gids), params)
    assert ei.value.overflow_flags & (1 << 10)
    assert "CUDA persistent subtree overflow" in ei.value.message
    assert "OVERSIZED_TERMINAL_NODE" in ei.value.message


def test_subtree_rejects_bad_root_leaders(gpu, orc):
    codes, scales, norms, gids = _data(orc, 500, 16, 4, 3)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, 16)
    params = S.PiPNNSubtreeParams(leaf_knn=8, c_max=256, fanout_second=2)
    with pytest.raises(N.TessaError) as ei:
        sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, root_leader_ids=np.array([3, 500])), params)
    assert "exceeds resident rows" in ei.value.message


def test_walk_equals_level_by_level_launches(gpu, orc):
    """The persistent walk (one cooperative launch for the whole level loop)
    and the level-by-level launches the capture path uses build the same
    leaves, top-k and counters (the walk's phase clocks aside), on a tree
    with retries, several levels and a balanced fallback-prone leader count."""
    codes, scales, norms, gids = _data(orc, 30000, 64, 12, 41)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, 64)
    params = S.PiPNNSubtreeParams(leaf_knn=16, c_max=256, psamp_fraction=0.0005, max_leaders=128, max_depth=64,
                                  fanout_second=2, random_seed=3)
    req = S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=90000, min_recurse_size=64)
    walk = sess.run(req, params)
    sess.set_assignment_capture(256)  # capture runs the partition level by level
    host = sess.run(req, params)
    sess.set_assignment_capture(0)
    torch.cuda.synchronize()
    assert walk.leaf_count == host.leaf_count and walk.leaf_rows == host.leaf_rows and walk.levels == host.levels
    lr, lc = walk.leaf_rows, walk.leaf_count
    assert torch.equal(walk.leaf_row_ids[:lr], host.leaf_row_ids[:lr])
    assert torch.equal(walk.leaf_starts[:lc], host.leaf_starts[:lc])
    assert torch.equal(walk.leaf_sizes[:lc], host.leaf_sizes[:lc])
    n = walk.leaf_rows * walk.k
    assert torch.equal(walk.topk_ids[:n], host.topk_ids[:n]) and torch.equal(walk.topk_dists[:n], host.topk_dists[:n])
    for w in range(N.SUBTREE_COUNTER_WORDS):
        if w not in N.P_CLOCK_WORDS:
            assert walk.counters[w] == host.counters[w], f"counter word {w}"
    assert walk.counters[N.P_LARGE_SPLIT_RETRIES] > 0 and walk.levels > 3
    # phase clocks: set by the walk, each phase inside the whole
    busy = int(walk.counters[N.P_PARTITION_BUSY_CLOCKS])
    assert busy > 0 and all(int(host.counters[w]) == 0 for w in N.P_CLOCK_WORDS)
    parts = [int(walk.counters[w]) for w in (N.P_LARGE_COUNT_DISTANCE_CLOCKS, N.P_LARGE_COUNT_COMMIT_CLOCKS,
                                              N.P_LARGE_SCATTER_CLOCKS, N.P_LARGE_PUBLISH_CLOCKS)]
    assert all(p > 0 for p in parts) and sum(parts) <= busy
    sess.close()
