"""CPU restatement of the whole graph build: the checker and CPU baseline of
shear_amd.pipeline.build_graph (test infrastructure only; nothing in the
product imports it).

Stage by stage it chains the oracle's restatements of the reference path
(paths relative to shear-core/src/algorithm/pipnn/ of SHEAR):

  quantize_sq_int8_matrix   dco_sq_int8.rs:1331-1467         orc_sq8_quantize
  global D0 assignment      compute_backend.rs:18016-18511   orc_d0_assign
  subtree partition         compute_backend.rs:12456-15727   orc_subtree_partition
  leaf top-k                leaf_build.rs:887-957            orc_leaf_topk_batch
  compact batches           compute_backend.rs:32243-32339   (restated below)
  record -> edge            leaf_build.rs:1679-1829          orc_flush_compact_topk_into_edges
  HashPrune reservoirs      hash_prune.rs:1243-1283          orc_hashprune_reduce
  (named R-half backfill)   hash_prune.rs:2601-2682          orc_hashprune_rhalf_reduce
  final RobustPrune (opt.)  pipnn_builder.rs:287-330         orc_robust_prune
  `_mem.index` image        pipnn_oom_writer.rs:23-72        graph_bytes
  entry point               rbc_partition.rs:4964-4985       (restated below)
  terminal-depth retry      rbc_partition.rs:3004-3017, :15066-15115 (restated below)

with the same inputs the GPU build takes (points, sketches, D0 leader rows,
parameters), so the two images must be equal byte for byte.  The only
product code it calls is the host-side plan arithmetic (leaf_min / leaf_max /
queue capacities, pinned by the reference's plan tests).
"""
from __future__ import annotations

import time

import numpy as np

from . import pyoracle as orc


def _plan(rows: int, leaf_knn: int, max_leaders: int, fanout: int, c_max: int):
    from shear_amd import subtree as S

    return S.plan_subtree(rows, leaf_knn, min(max_leaders, 128), fanout, None, c_max)


def entry_point(child_offsets, child_points) -> int:
    """rbc_partition.rs:4964-4985: first point of the largest child, ties to
    the smaller point id."""
    best = None
    for c in range(len(child_offsets) - 1):
        a, b = int(child_offsets[c]), int(child_offsets[c + 1])
        if b > a:
            cand = (b - a, -int(child_points[a]))
            best = cand if best is None or cand > best else best
    return -best[1] if best is not None else 0


def build_graph_cpu(x: np.ndarray, sketches: np.ndarray, leader_rows: np.ndarray, p, threads: int = 0):
    """-> dict(image bytes, start, rows (neighbour lists), build_s, stages).
    ``p`` is a shear_amd.pipeline.GraphBuildParams (plain numbers)."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.shape[0]
    w0 = time.perf_counter()
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(rows, dtype=np.uint32)
    lr = np.asarray(leader_rows, np.int64)
    _, offs, pts = orc.d0_assign(codes, scales, norms, gids, codes[lr], scales[lr], norms[lr],
                                 gids[lr], p.fanout_top)
    start = entry_point(offs, pts)
    w1 = time.perf_counter()
    parts = []
    leaves_n = leaf_rows_n = retries = 0
    for c in range(len(offs) - 1):
        a, b = int(offs[c]), int(offs[c + 1])
        if b - a < 2:
            continue
        cg = pts[a:b].astype(np.uint32)
        cc, cs, cn = codes[cg], scales[cg], norms[cg]
        n = b - a
        seed = orc.subtree_root_seed(p.random_seed, 1, n, rows, p.min_recurse_size)
        plan = _plan(n, p.leaf_knn, p.max_leaders, p.fanout_second, p.c_max)
        def part(max_depth):
            return orc.subtree_partition(cc, cs, cn, seed=seed, root_depth=1, max_depth=max_depth,
                                         max_leaders=min(p.max_leaders, 128), fanout_second=p.fanout_second,
                                         leaf_min=plan.leaf_min, leaf_max=plan.leaf_max,
                                         psamp_fraction=p.psamp_fraction, max_leaf_count=plan.max_leaf_count,
                                         max_leaf_rows=plan.max_leaf_rows)

        leaves, ctr = part(p.max_depth)
        if leaves is None and int(ctr[7]) == 1 << 10:
            # rbc_partition.rs:3004-3017, :15066-15115: one retry with max_depth >= 1024
            leaves, ctr = part(max(p.max_depth + 1, 1024))
            retries += 1
        if leaves is None:
            raise RuntimeError(f"oracle partition of D0 child {c} overflowed: flags 0x{int(ctr[7]):x}")
        sizes = np.array([len(lf) for lf in leaves], np.int64)
        members = np.concatenate(leaves).astype(np.uint32)
        loffs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
        k = p.leaf_knn
        ids, d = orc.leaf_topk(cc, cs, cn, cg, members, loffs, sizes, k, threads=threads)
        ids = ids.reshape(-1, k)
        d = d.reshape(-1, k)
        # compact batches (compute_backend.rs:32243-32339): per leaf k_eff =
        # min(leaf_knn, size - 1) slots of each row; then the leaf's records
        for lf, a2, sz in zip(leaves, loffs.tolist(), sizes.tolist()):
            ke = min(k, max(sz - 1, 0))
            if ke == 0:
                continue
            parts.append(orc.flush_compact_topk_into_edges(cg[lf], ke, ids[a2:a2 + sz, :ke].reshape(-1),
                                                           d[a2:a2 + sz, :ke].reshape(-1), sketches, p.m_hash_bits))
        leaves_n += len(leaves)
        leaf_rows_n += int(sizes.sum())
    records = np.concatenate(parts) if parts else np.zeros(0, orc.EDGE_DTYPE)
    w2 = time.perf_counter()
    bf = getattr(p, "hashprune_backfill", None)
    if bf is not None and bf.mode != "off":
        t, _, _, cnt, _ = orc.hashprune_rhalf_reduce(rows, p.l_max, records, mode=bf.mode,
                                                     hash_quota=bf.hash_quota or 0,
                                                     row_cap=bf.max_backfill_per_row or 0,
                                                     priority_alpha=bf.soft_tier_priority_alpha or 0.0)
    else:
        t, _, _, cnt = orc.hashprune_reduce(rows, p.l_max, records)
    if getattr(p, "final_prune", False):
        t, cnt = orc.robust_prune(x, t, cnt, p.l_max, p.prune_max_occlusion, p.prune_alpha, p.prune_saturate)
    nbr = [t[i, : cnt[i]] for i in range(rows)]
    image = orc.graph_bytes(start, 0, nbr)
    w3 = time.perf_counter()
    stages = {"quantize_d0_s": round(w1 - w0, 3), "subtrees_and_records_s": round(w2 - w1, 3),
              "hashprune_and_image_s": round(w3 - w2, 3), "leaves": leaves_n, "leaf_rows": leaf_rows_n,
              "edge_records": int(len(records)), "terminal_depth_retries": retries}
    return {"image": image, "start": start, "rows": nbr, "build_s": w3 - w0, "stages": stages}
