"""Asynchronous subtree submissions (tessa_session_submit_subtree / wait /
release, the reference's submit_owned_quantized_subtree_l2_compact_topk with
its pinned host-slot ring): results identical to the synchronous call and to
the oracle; slot ring and error behaviour."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import _native as N
from shear_amd import datagen
from shear_amd import subtree as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _task(orc, n, dim, seed):
    x = datagen.gmm_numpy(n, dim, 8, 0.3, seed)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(seed).permutation(1 << 20)[:n].astype(np.uint32)
    return codes, scales, norms, gids


def _params(**kw):
    base = dict(leaf_knn=16, c_max=256, psamp_fraction=0.01, fanout_second=2, random_seed=11)
    base.update(kw)
    return S.PiPNNSubtreeParams(**base)


def _same_batches(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert x.leaf_id == y.leaf_id and x.rows == y.rows and x.k == y.k
        assert np.array_equal(x.point_ids, y.point_ids)
        assert np.array_equal(x.topk_ids, y.topk_ids)
        assert np.array_equal(x.topk_dists.view(np.uint32), y.topk_dists.view(np.uint32))


def test_deferred_results_match_synchronous_runs(gpu, orc):
    tasks = [_task(orc, n, 40, 100 + n) for n in (2500, 1200, 3100)]
    params = _params()
    sess = S.SubtreeSession(0)
    # two in flight, then a third once the first is finished (slot ring of 2)
    req = [S.GpuSubtreePartitionRequest(point_ids=t[3], parent_points=3 * len(t[3])) for t in tasks]
    d0 = sess.submit_owned_quantized_subtree_l2_compact_topk(req[0], *tasks[0], 40, params)
    d1 = sess.submit_owned_quantized_subtree_l2_compact_topk(req[1], *tasks[1], 40, params)
    r0 = d0.finish()
    d2 = sess.submit_owned_quantized_subtree_l2_compact_topk(req[2], *tasks[2], 40, params)
    r1, r2 = d1.finish(), d2.finish()
    for t, q, r in zip(tasks, req, (r0, r1, r2)):
        ref = S.SubtreeSession(0)
        ref.upload(*t, 40)
        want = ref.process_quantized_subtree_l2_compact_topk(q, params)
        ref.close()
        _same_batches(r.compact_batches, want.compact_batches)
        assert r.leaf_count == want.leaf_count and r.assignment_passes == want.assignment_passes
    # and the first task against the oracle
    codes, scales, norms, gids = tasks[0]
    seed = S.subtree_root_seed(11, 0, len(gids), 3 * len(gids), 64)
    plan = S.plan_subtree(len(gids), 16, 128, 2, None, 256)
    leaves, ctr = orc.subtree_partition(codes, scales, norms, seed=seed, fanout_second=2, leaf_min=plan.leaf_min,
                                        leaf_max=plan.leaf_max, psamp_fraction=0.01,
                                        max_leaf_count=plan.max_leaf_count, max_leaf_rows=plan.max_leaf_rows)
    assert [list(b.point_ids) for b in r0.compact_batches] == [list(gids[x]) for x in leaves]
    members = np.concatenate(leaves).astype(np.uint32)
    sizes = [len(x) for x in leaves]
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members,
                                     np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64), sizes, 16)
    got_ids = np.concatenate([b.topk_ids.reshape(b.rows, b.k) for b in r0.compact_batches]).reshape(-1)
    got_d = np.concatenate([b.topk_dists.reshape(b.rows, b.k) for b in r0.compact_batches]).reshape(-1)
    assert np.array_equal(got_ids, want_ids) and np.array_equal(got_d.view(np.uint32), want_d.view(np.uint32))
    sess.close()


def test_slot_ring_is_bounded_and_released(gpu, orc):
    t = _task(orc, 800, 24, 5)
    params = _params()
    q = S.GpuSubtreePartitionRequest(point_ids=t[3], parent_points=2400)
    sess = S.SubtreeSession(0)
    d0 = sess.submit_owned_quantized_subtree_l2_compact_topk(q, *t, 24, params)
    d1 = sess.submit_owned_quantized_subtree_l2_compact_topk(q, *t, 24, params)
    with pytest.raises(N.TessaError, match="both pinned host result slots are held"):
        sess.submit_owned_quantized_subtree_l2_compact_topk(q, *t, 24, params)
    a, b = d0.finish(), d1.finish()
    _same_batches(a.compact_batches, b.compact_batches)
    d2 = sess.submit_owned_quantized_subtree_l2_compact_topk(q, *t, 24, params)  # slots are free again
    _same_batches(d2.finish().compact_batches, a.compact_batches)
    with pytest.raises(N.TessaError, match="no pending or unreleased submission"):
        d2.finish()  # already released
    sess.close()


def test_deferred_error_is_reported_by_finish(gpu, orc):
    t = _task(orc, 1500, 16, 3)
    sess = S.SubtreeSession(0)
    bad = _params(leaf_knn=8, c_max=100, psamp_fraction=0.002, max_depth=1, fanout_second=1)
    d = sess.submit_owned_quantized_subtree_l2_compact_topk(S.GpuSubtreePartitionRequest(point_ids=t[3]), *t, 16,
                                                            bad)
    with pytest.raises(N.TessaError) as e:
        d.finish()
    assert "CUDA persistent subtree overflow" in e.value.message
    assert "OVERSIZED_TERMINAL_NODE" in e.value.message
    # the session keeps working after a failed job
    ok = sess.submit_owned_quantized_subtree_l2_compact_topk(S.GpuSubtreePartitionRequest(point_ids=t[3]), *t, 16,
                                                             _params())
    assert ok.finish().leaf_count > 1
    sess.close()


def test_synchronous_calls_wait_for_a_running_job(gpu, orc):
    t = _task(orc, 3000, 32, 9)
    params = _params()
    q = S.GpuSubtreePartitionRequest(point_ids=t[3], parent_points=9000)
    sess = S.SubtreeSession(0)
    d = sess.submit_owned_quantized_subtree_l2_compact_topk(q, *t, 32, params)
    out = sess.run(q, params)  # same upload (the job's rows): queued behind the job
    torch.cuda.synchronize()
    r = d.finish()
    assert out.leaf_count == r.leaf_count
    rows = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
    assert np.array_equal(np.concatenate([b.point_ids for b in r.compact_batches]), t[3][rows])
    sess.close()
