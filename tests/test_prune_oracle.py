"""Pins of the final RobustPrune oracle (oracle/tessa_prune.c) by hand-worked
occlusions (shear-core/src/algorithm/prune/prune.rs:17-214,
index/inmem_index/pipnn_builder.rs:287-330)."""
import numpy as np
import pytest


def table(rows, stride):
    t = np.full((len(rows), stride), 0xFFFFFFFF, np.uint32)
    c = np.zeros(len(rows), np.uint32)
    for p, r in enumerate(rows):
        t[p, :len(r)] = r
        c[p] = len(r)
    return t, c


def prune_row0(orc, pts, nbrs, **kw):
    x = np.asarray(pts, np.float32)
    rows = [nbrs] + [[] for _ in range(len(x) - 1)]
    t, c = table(rows, max(len(nbrs), 1))
    out, cnt = orc.robust_prune(x, t, c, **kw)
    return out[0, :cnt[0]].tolist(), cnt


def test_point_behind_a_kept_one_is_dropped(orc):
    # node 0 at the origin; 1, 2, 3 on one ray: 1 is kept, 2 and 3 are occluded
    # (d(0,2)/d(2,1) = 4, d(0,3)/d(3,1) = 2.25, both > 1.2)
    got, _ = prune_row0(orc, [[0, 0], [1, 0], [2, 0], [3, 0]], [3, 1, 2])
    assert got == [1]


def test_orthogonal_points_are_both_kept(orc):
    # factor d(0,2)/d(2,1) = 1/2 <= 1
    got, _ = prune_row0(orc, [[0, 0], [1, 0], [0, 1]], [2, 1])
    assert got == [1, 2]


def test_second_alpha_pass(orc):
    # b = (0.9, sqrt(7.99)): |b|^2 = 8.8, |b - a|^2 = 8.0, factor 1.1: waits in the
    # 1.0 pass, is taken in the 1.2 pass; with alpha 1.0 it never is
    b = [0.9, float(np.sqrt(np.float32(7.99)))]
    pts = [[0, 0], [1, 0], b]
    assert prune_row0(orc, pts, [2, 1])[0] == [1, 2]
    assert prune_row0(orc, pts, [2, 1], alpha=1.0)[0] == [1]
    # with a cap of one neighbour the second pass never runs
    assert prune_row0(orc, pts, [2, 1], max_degree=1)[0] == [1]


def test_self_loop_and_duplicates(orc):
    # the node itself sorts first (distance 0) and is not emitted, but occludes
    # with factor d_j / d_j = 1 (not > 1.0, so nothing is dropped by it); a
    # coincident copy of a kept point has distance 0 to it and is dropped
    got, _ = prune_row0(orc, [[0, 0], [1, 0], [0, 1], [1, 0]], [0, 3, 1, 2])
    assert got == [1, 2]


def test_saturate_and_empty_rows(orc):
    pts = [[0, 0], [1, 0], [2, 0], [3, 0]]
    assert prune_row0(orc, pts, [3, 1, 2], saturate=True)[0] == [1, 2, 3]
    assert prune_row0(orc, pts, [3, 1, 2], saturate=True, alpha=1.0)[0] == [1]  # only with alpha > 1
    got, cnt = prune_row0(orc, pts, [])
    assert got == [] and cnt.tolist() == [0, 0, 0, 0]


def test_occlusion_cap_truncates_the_sorted_pool(orc):
    pts = [[0, 0], [1, 0], [0, 2], [-3, 0]]
    assert prune_row0(orc, pts, [3, 2, 1], max_occlusion=2)[0] == [1, 2]
    assert prune_row0(orc, pts, [3, 2, 1])[0] == [1, 2, 3]
