"""Many-root partition (tessa_session_partition_roots) against one subtree
run per root: on the C1 mixture's D0 children (and on tight clusters that
take the terminal-depth retry) every root's leaves, as lists of SQ8 rows in
member order, equal those of the root's own run; the whole build writes the
same `_mem.index` image with and without many-root runs."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import d0 as D
from shear_amd import datagen
from shear_amd import pipeline as P
from shear_amd import subtree as S
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu


def _children(x, p, leaders):
    gpu = require_gpu()
    xd = torch.from_numpy(x).to(gpu)
    sq8 = T.quantize_sq_int8_matrix(xd)
    rows = sq8.rows
    gids = torch.arange(rows, dtype=torch.int32, device=gpu)
    lr = torch.from_numpy(P.d0_leader_rows(rows, leaders, p.random_seed)).to(gpu)
    lead = T.Sq8Matrix(sq8.codes[lr].contiguous(), sq8.scales[lr].contiguous(), sq8.norms[lr].contiguous(), sq8.dim)
    _, _, offs, pts = D.global_d0_assign(sq8, gids, lead, gids[lr].contiguous(), p.fanout_top)
    return sq8, gids, offs.cpu().numpy(), pts


def _per_root_leaves(sess, sq8, pts, offs, roots, rows, p, max_depth):
    sp = P.replace(p.subtree_params(), max_depth=max_depth)
    out = []
    for c in roots:
        a, b = int(offs[c]), int(offs[c + 1])
        cg = pts[a:b]
        ci = cg.long()
        sess.upload_device(T.Sq8Matrix(sq8.codes[ci], sq8.scales[ci], sq8.norms[ci], sq8.dim), cg)
        r = sess.run(S.GpuSubtreePartitionRequest(point_ids=np.zeros(b - a, np.uint32), depth=1, parent_points=rows,
                                                  min_recurse_size=p.min_recurse_size), sp, partition_only=True)
        g = cg.cpu().numpy().view(np.uint32)
        li = r.leaf_row_ids[: r.leaf_rows].cpu().numpy().view(np.uint32)
        st = r.leaf_starts[: r.leaf_count].cpu().numpy()
        sz = r.leaf_sizes[: r.leaf_count].cpu().numpy()
        out.append(sorted(tuple(g[li[s:s + n]].tolist()) for s, n in zip(st, sz)))
    return out


def _many_root_leaves(sess, sq8, pts, offs, roots, rows, p, max_depth):
    rows_t = torch.cat([pts[int(offs[c]):int(offs[c + 1])] for c in roots])
    roffs = np.zeros(len(roots) + 1, np.uint64)
    roffs[1:] = np.cumsum([int(offs[c + 1] - offs[c]) for c in roots])
    seeds = np.array([S.subtree_root_seed(p.random_seed, 1, int(offs[c + 1] - offs[c]), rows, p.min_recurse_size)
                      for c in roots], np.uint64)
    ro = sess.partition_roots(sq8, rows_t, roffs, seeds, p.subtree_params(), depth=1, max_depth=max_depth)
    lc = ro.leaf_count
    lr = ro.leaf_rows[: ro.leaf_rows_total].cpu().numpy().view(np.uint32)
    st = ro.leaf_starts[:lc].cpu().numpy()
    sz = ro.leaf_sizes[:lc].cpu().numpy()
    rt = ro.leaf_roots[:lc].cpu().numpy()
    dp = ro.leaf_depths[:lc].cpu().numpy()
    per = [[] for _ in roots]
    deepest = np.zeros(len(roots), np.int64)
    for s, n, r, d in zip(st, sz, rt, dp):
        per[r].append(tuple(lr[s:s + n].tolist()))
        deepest[r] = max(deepest[r], d)
    return [sorted(v) for v in per], deepest, ro


def test_many_root_leaves_equal_per_root_runs_c1():
    x, _ = datagen.c1_numpy()
    p = P.GraphBuildParams()
    sq8, gids, offs, pts = _children(x, p, P.d0_leader_count(x.shape[0], x.shape[1], p))
    sizes = np.diff(offs)
    roots = [c for c in range(len(sizes)) if sizes[c] > max(256, p.c_max)]
    assert len(roots) > 50
    sess = S.SubtreeSession(0)
    want = _per_root_leaves(sess, sq8, pts, offs, roots, sq8.rows, p, p.max_depth)
    got, deepest, ro = _many_root_leaves(sess, sq8, pts, offs, roots, sq8.rows, p, p.max_depth)
    for i, c in enumerate(roots):
        assert got[i] == want[i], f"root {i} (D0 child {c}): leaves differ"
    assert ro.leaf_rows_total == sum(sum(len(lf) for lf in w) for w in want)
    assert int(deepest.max()) <= p.max_depth


def test_many_root_retry_depths_match_per_root_runs():
    # tight clusters under max_depth 2: a root's run fails at max_depth 2 iff one of its many-root leaves
    # lies deeper than 2; those roots' leaves equal their run at max_depth 1024
    x = datagen.gmm_numpy(20000, 64, 4, 0.05, 5)
    p = P.GraphBuildParams(max_depth=2, c_max=256)
    sq8, gids, offs, pts = _children(x, p, 8)
    sizes = np.diff(offs)
    roots = [c for c in range(len(sizes)) if sizes[c] > 256]
    sess = S.SubtreeSession(0)
    got, deepest, _ = _many_root_leaves(sess, sq8, pts, offs, roots, sq8.rows, p, 1024)
    want = _per_root_leaves(sess, sq8, pts, offs, roots, sq8.rows, p, 1024)
    assert got == want
    failed = []
    for c in roots:
        try:
            _per_root_leaves(sess, sq8, pts, offs, [c], sq8.rows, p, 2)
            failed.append(False)
        except Exception as e:  # OVERSIZED_TERMINAL_NODE
            assert "OVERSIZED_TERMINAL_NODE" in str(e)
            failed.append(True)
    assert any(failed)
    assert failed == [bool(d > 2) for d in deepest]


def test_build_image_same_with_and_without_many_root_runs():
    gpu = require_gpu()
    x, _ = datagen.c1_numpy()
    rows, dim = x.shape
    xd = torch.from_numpy(x).to(gpu)
    p = P.GraphBuildParams()
    sk = torch.from_numpy(P.sketches_of(x, P.sketch_planes(dim, p.m_hash_bits, 7))).to(gpu)
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    many = P.build_graph(xd, sk, lead, p)
    one = P.build_graph(xd, sk, lead, P.replace(p, multi_root=False))
    assert many.stages["multi_root_children"] > 0 and one.stages["multi_root_children"] == 0
    assert many.stages["edge_records"] == one.stages["edge_records"]
    assert torch.equal(many.image, one.image)
    print(f"C1 build: many-root {many.build_s * 1e3:.1f} ms (partition {many.stages['partition_ms']} ms), "
          f"per child {one.build_s * 1e3:.1f} ms (partition {one.stages['partition_ms']} ms)")
