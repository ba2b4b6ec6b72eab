"""End-to-end PiPNN graph build with the subtree operator on the GPU.

Host mirror of SHEAR's build with the CUDA subtree backend (paths relative to
shear-core/src/algorithm/pipnn/):

* ``build_graph``             build_pipnn_graph_with_store (mod.rs:3365) as it runs
  with ``--pipnn-backend cuda``: SQ8 payload, global D0 assignment
  (rbc_partition.rs:7174 rbc_partition_gpu_subtree_streaming), one subtree
  task per D0 child through the operator (process_quantized_subtree_l2_compact_topk,
  compute_backend.rs:3794-3805; child depth 1, so its root uses fanout_second),
  candidate records -> edge records (leaf_build.rs:1679-1829) -> HashPrune
  reservoirs (hash_prune.rs:1243-1283, l_max = R), optionally the final
  RobustPrune (pipnn_builder.rs:149, :199-225, :287-330), then the
  `_mem.index` image (pipnn_oom_writer.rs:23-72)
* ``entry_point``             gpu_subtree_entry_point_from_sq_payloads
  (rbc_partition.rs:4964-4985): the first point of the largest D0 child, ties
  to the smaller point id
* ``GraphBuildParams``        the PiPNNParams fields this path reads (params.rs:2109-2111
  fanout_top / fanout_second, :3341-3370 defaults); ``hashprune_backfill``
  the named R-half policy (params.rs:2070-2083), off as in PiPNNParams'
  default, ``hashprune.PRODUCTION_BACKFILL`` for the build_shear_index
  binary's SoftTier-Q3 cap 3 (main.rs:2360-2374)

The final RobustPrune follows the build_shear_index binary: it runs only when
asked (``final_prune``, the binary's ``--final-prune`` flag, off unless given:
apps/build_shear_index/src/main.rs:3752-3754, copied into PiPNNParams at
:4006 / :4064, although PiPNNParams::default() sets it, params.rs:3491), over
the f32 points with the binary's write parameters (alpha 1.2 and max
occlusion 750 from the builder defaults, index_write_parameters.rs:8, :17;
saturate on, main.rs:3004-3007).  ``final_prune_alpha`` (params.rs:2372) is
read by nothing in the reference; the prune's alpha is the write
parameters' alpha, ``prune_alpha`` here.

Every stage runs in libtessa_hip.so; this module orders the calls.  The D0
leader sample and the sketch hyperplanes are inputs (the reference draws both
with rand's StdRng, which this build does not reproduce), so a CPU build fed
the same inputs must produce the same image byte for byte.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field, replace

import numpy as np
import torch

from . import d0 as D
from . import edges as E
from . import graph as G
from . import hashprune as H
from . import subtree as S
from . import tessa as T
from . import _native as N
from . import tierlift as TL

# rbc_partition.rs:3004-3017: a D1+ child whose run fails with exactly
# OVERSIZED_TERMINAL_NODE is run once more, unchanged but for max_depth =
# max(max_depth + 1, 1024).
OVF_OVERSIZED_TERMINAL_NODE = 1 << 10
TERMINAL_DEPTH_RECOVERY_FLOOR = 1024
TERMINAL_DEPTH_RETRY_LIMIT = 1
SMALL_NODE_LIMIT = 4096  # the plan's small-node scratch rows (compute_backend.rs:1341)


@dataclass
class GraphBuildParams:
    fanout_top: int = 2        # D0 replication: each point to its fanout_top nearest leaders
    fanout_second: int = 2     # replication at each subtree's root (depth 1)
    c_max: int = 1024          # leaf size bound (plan leaf_max = max(256, c_max))
    leaf_knn: int = 32         # k of the leaf top-k
    l_max: int = 64            # HashPrune reservoir = maximum out-degree R
    m_hash_bits: int = 12
    psamp_fraction: float = 0.001
    max_leaders: int = 128
    max_depth: int = 16
    random_seed: int = 42
    min_recurse_size: int = 64
    multi_root: bool = True    # large D0 children partitioned together (tessa_session_partition_roots)
    roots_rows_per_run: int = 1 << 26  # rows of the children partitioned by one many-root run
    leaf_chunk_rows: int = 1 << 22     # leaf rows per leaf top-k / record batch of a many-root run
    gpu_workspace_budget_bytes: int = 0  # per subtree task (0: the default 512 MiB plan, tasks unchecked)
    final_prune: bool = False      # build_shear_index --final-prune (off unless given)
    final_prune_alpha: float = 1.2  # PiPNNParams field, unused by the reference's prune
    prune_alpha: float = 1.2        # write parameters' alpha: what the final prune uses
    prune_max_occlusion: int = 750
    prune_saturate: bool = True     # build_shear_index builds its write parameters with saturate_graph(true)
    hashprune_backfill: H.HashPruneBackfill | None = None  # named R-half policy (None: off)
    # device reservoirs: leave the repeats of mutual pairs out of the emitted
    # records (same reservoirs; 16-17 % fewer records to merge, but the
    # emission's list lookups cost more than the merge saves: C3 0.42-0.46 s
    # with, 0.38-0.43 s without)
    drop_mutual_repeats: bool = False

    def subtree_params(self) -> S.PiPNNSubtreeParams:
        return S.PiPNNSubtreeParams(leaf_knn=self.leaf_knn, c_max=self.c_max, fanout_second=self.fanout_second,
                                    psamp_fraction=self.psamp_fraction, max_leaders=self.max_leaders,
                                    random_seed=self.random_seed, max_depth=self.max_depth)


def d0_leader_count(rows: int, dim: int, p: GraphBuildParams) -> int:
    """D0 leaders: the capacity plan's count (largest admitted subtree under the
    default 512 MiB workspace) or the sampling-rate count, whichever is larger
    (the plan alone asks for its quality floor of 64 at 200k points, whose
    ~6k-row children are fine, but the sampling rate keeps children near the
    reference's expected size)."""
    budget = p.gpu_workspace_budget_bytes or D.DEFAULT_GPU_WORKSPACE_BUDGET_BYTES
    c_gpu = D.find_max_admissible_rows(dim, p.leaf_knn, min(p.max_leaders, D.GPU_QUEUE_LEADER_STRIDE),
                                       p.fanout_second, budget, None, p.c_max)
    plan = D.plan_root_leaders(rows, p.fanout_top, D.compute_thresholds(c_gpu))
    return min(rows, max(int(plan["k_initial"]), D.d0_leader_count(rows)))


def d0_leader_rows(rows: int, count: int, seed: int) -> np.ndarray:
    """``count`` distinct rows of [0, rows), ascending (int64)."""
    return D.sample_leader_rows(rows, count, seed, "cpu").numpy()


def sketch_planes(dim: int, m_bits: int, seed: int) -> np.ndarray:
    """m_bits hyperplanes with coordinates uniform in [-1, 1) (f32, [m_bits, dim])."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return (torch.rand((m_bits, dim), generator=g) * 2.0 - 1.0).numpy()


def sketches_of(x: np.ndarray, planes: np.ndarray) -> np.ndarray:
    """Per-point sketch coordinates (f32 [rows, m_bits]): f64 dot products
    rounded to f32, computed once on the host and handed to every build of
    the same points (the reference's SketchAccessor rows)."""
    return (np.asarray(x, np.float64) @ np.asarray(planes, np.float64).T).astype(np.float32)


def sq8_from_chunks(chunks, rows: int, dim: int, planes: torch.Tensor):
    """(Sq8Matrix, sketches f32 [rows, m_bits]) of a point set produced as f32
    device chunks in row order: each chunk is quantized (SQ8 is per vector)
    and sketched against ``planes`` (device f32 [m_bits, dim]) as it arrives,
    so the f32 set is never resident as a whole."""
    dev = planes.device
    pd = T.sq_int8_padded_dim(dim)
    codes = torch.empty((rows, pd), dtype=torch.int8, device=dev)
    scales = torch.empty(rows, dtype=torch.float32, device=dev)
    norms = torch.empty(rows, dtype=torch.float32, device=dev)
    sk = torch.empty((rows, planes.shape[0]), dtype=torch.float32, device=dev)
    at = 0
    for x in chunks:
        m = x.shape[0]
        if at + m > rows or x.shape[1] != dim:
            raise ValueError(f"chunk of shape {tuple(x.shape)} at row {at} does not fit [{rows}, {dim}]")
        q = T.quantize_sq_int8_matrix(x)
        codes[at:at + m] = q.codes
        scales[at:at + m] = q.scales
        norms[at:at + m] = q.norms
        sk[at:at + m] = x @ planes.t()
        at += m
        del q, x
    if at != rows:
        raise ValueError(f"chunks held {at} rows, expected {rows}")
    return T.Sq8Matrix(codes, scales, norms, dim), sk


def entry_point(child_offsets: np.ndarray, child_points: np.ndarray) -> int:
    """First point of the largest D0 child (ties: the smaller point id)."""
    offs = np.asarray(child_offsets, np.int64)
    sizes = np.diff(offs)
    firsts = np.zeros(len(sizes), np.int64)
    nz = np.nonzero(sizes > 0)[0]
    firsts[nz] = np.asarray(child_points)[offs[nz]]
    return _entry_point_of(sizes, firsts)


def _entry_point_of(sizes: np.ndarray, firsts: np.ndarray) -> int:
    """entry_point from the child sizes and each non-empty child's first point."""
    best = None
    for c in np.nonzero(sizes > 0)[0]:
        cand = (int(sizes[c]), -int(firsts[c]))
        if best is None or cand > best:
            best = cand
    return -best[1] if best is not None else 0


@dataclass
class BuiltGraph:
    targets: torch.Tensor   # int32 [rows, l_max] (row p's neighbours first, ascending hash)
    counts: torch.Tensor    # int32 [rows]
    start: int
    image: torch.Tensor     # uint8 `_mem.index` image (device)
    build_s: float
    stages: dict = field(default_factory=dict)


def run_child(sess: S.SubtreeSession, req: S.GpuSubtreePartitionRequest, sp: S.PiPNNSubtreeParams):
    """One D0 child's subtree run with the reference's terminal-depth retry
    (rbc_partition.rs:15066-15115); the output's ``retried`` tells whether it
    took the retry."""
    try:
        out = sess.run(req, sp)
        out.retried = False
        return out
    except N.TessaError as e:
        if e.overflow_flags != OVF_OVERSIZED_TERMINAL_NODE:
            raise
        nxt = max(sp.max_depth + 1, TERMINAL_DEPTH_RECOVERY_FLOOR)
        if nxt == sp.max_depth:
            raise
    out = sess.run(req, replace(sp, max_depth=nxt))
    out.retried = True
    return out


def build_graph(x: torch.Tensor, sketches: torch.Tensor, leader_rows: np.ndarray,
                p: GraphBuildParams = GraphBuildParams(), observer=None,
                host_reducer: TL.TierLiftParams | None = None) -> BuiltGraph:
    """Build the graph of the f32 rows ``x`` (device tensor [rows, dim]).

    ``sketches`` (device f32 [rows, m_bits]) and ``leader_rows`` (ascending
    resident rows) are the build's inputs; global ids are the row numbers."""
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    sq8 = T.quantize_sq_int8_matrix(x)
    return build_graph_sq8(sq8, sketches, leader_rows, p, observer, t0=w0, host_reducer=host_reducer,
                           points=x if p.final_prune else None)


def build_graph_sq8(sq8: T.Sq8Matrix, sketches: torch.Tensor, leader_rows: np.ndarray,
                    p: GraphBuildParams = GraphBuildParams(), observer=None,
                    t0: float | None = None, host_reducer: TL.TierLiftParams | None = None,
                    points: torch.Tensor | None = None) -> BuiltGraph:
    """The build from an SQ8 payload already in device memory (build time
    counted from ``t0``, a perf_counter value, when given).  ``points`` (the
    f32 rows on the device) is needed only for ``p.final_prune``.

    D0 children of two or more points are the subtree tasks.  With
    ``p.multi_root`` (the default) every large child (more than leaf_max rows,
    or a fanout probe beyond the small-node scratch) is partitioned in one
    many-root run per group of about ``p.roots_rows_per_run`` rows, reading
    the SQ8 rows in place; the leaves of a group then go through the leaf
    top-k and record emission in chunks of at most ``p.leaf_chunk_rows`` leaf
    rows.  The remaining small children run one by one.  Each child's leaves
    are those of its own run, so the graph is the same either way.

    ``observer`` (optional) is called after each batch of records is emitted,
    as observer(tag, global_ids, output, layouts, records, record_count,
    segments, segment_count): ``output`` has leaf_row_ids / leaf_starts /
    leaf_sizes / leaf_count / leaf_rows / k / topk_ids / topk_dists of the
    batch (starts relative to its leaf_row_ids) and ``global_ids`` maps its
    rows to point ids (None: the rows are point ids); ``segments`` is None
    when the records go to TierLift; it must not keep device tensors alive.

    For the device reservoirs the records are emitted source-grouped, with
    ``p.drop_mutual_repeats`` without the repeats of mutual pairs
    (edges.emit_edge_segments(unique=True): the reverse record of a slot whose
    target lists the source at the same distance is that target's forward
    record); the reservoirs, a function of the record set, are the same
    either way.

    ``host_reducer`` routes the records through the TierLift host reducer
    (bounded host memory, spill files past the budget) instead of device
    reservoirs: each batch of records is queued for copy as soon as it is
    emitted, and the copies overlap the next batches' work.  Both reducers
    give the same table."""
    dev = sq8.codes.device
    rows = sq8.rows
    if p.final_prune and (points is None or tuple(points.shape) != (rows, sq8.dim)):
        raise ValueError("final_prune needs the f32 points [rows, dim] on the device")
    gids = torch.arange(rows, dtype=torch.int32, device=dev)
    lrows = torch.from_numpy(np.asarray(leader_rows, np.int64)).to(dev)
    torch.cuda.synchronize()
    w0 = t0 if t0 is not None else time.perf_counter()
    lead = T.Sq8Matrix(sq8.codes[lrows].contiguous(), sq8.scales[lrows].contiguous(),
                       sq8.norms[lrows].contiguous(), sq8.dim)
    _, _, offs, pts = D.global_d0_assign(sq8, gids, lead, gids[lrows].contiguous(), p.fanout_top)
    del lead
    offs_h = offs.cpu().numpy()
    # the entry point needs each child's first point only (not the whole point list)
    osz = np.diff(offs_h.astype(np.int64))
    fidx = torch.from_numpy(np.minimum(offs_h[:-1].astype(np.int64), max(pts.numel() - 1, 0))).to(dev)
    firsts = pts[fidx].cpu().numpy().view(np.uint32) if pts.numel() else np.zeros(len(osz), np.uint32)
    start = _entry_point_of(osz, firsts)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()  # the library allocates the reservoirs and workspaces itself, outside torch's cache
    w1 = time.perf_counter()
    sess = S.SubtreeSession(0)
    hp = tl = None
    if host_reducer is not None:
        if not host_reducer.expected_records:
            # each point in about fanout_top * fanout_second leaves, 2 * k records per leaf row
            host_reducer = replace(host_reducer, expected_records=rows * 2 * p.leaf_knn * max(p.fanout_top, 1)
                                   * max(p.fanout_second, 1))
        tl = TL.TierLiftReducer(rows, p.l_max, host_reducer, dev)
    else:
        hp = H.HashPruneReducer(rows, p.l_max, dev, p.hashprune_backfill)
    st = {"push_s": 0.0, "part_ms": 0.0, "leaf_ms": 0.0, "records": 0, "leaves": 0, "leaf_rows": 0,
          "retries": 0, "runs": 0, "emit_s": 0.0, "reduce_s": 0.0}
    sp = p.subtree_params()
    leaf_max = max(256, p.c_max)
    famp = max(p.fanout_second, 1)

    def emit(lay_gids, lay, k, ids, d):
        # device reservoirs merge source-grouped segments in place (repeats
        # of mutual pairs left out); TierLift routes records by source, in
        # any order, and drops repeats itself
        if tl is not None:
            rec, cnt = E.emit_edge_records(lay_gids, lay, k, ids, d, sketches, p.m_hash_bits)
            return rec, cnt, None, 0
        return E.emit_edge_segments(lay_gids, lay, k, ids, d, sketches, p.m_hash_bits,
                                    unique=p.drop_mutual_repeats)

    def consume(rec, cnt, segs, nseg):
        if tl is not None:
            q0 = time.perf_counter()
            tl.push(rec, int(cnt))
            st["push_s"] += time.perf_counter() - q0
        else:
            hp.insert_segments(rec, segs, nseg)

    sizes = np.diff(offs_h.astype(np.int64))
    children = [c for c in range(len(sizes)) if sizes[c] >= 2]  # a one-point child has no leaf pairs
    if p.multi_root:
        large = [c for c in children if sizes[c] > leaf_max or (famp > 1 and sizes[c] * famp > SMALL_NODE_LIMIT)]
    else:
        large = []
    large_set = set(large)
    small = [c for c in children if c not in large_set]

    # many-root runs over groups of large children
    group, group_rows = [], 0
    for gi, c in enumerate(large):
        group.append(c)
        group_rows += int(sizes[c])
        if gi + 1 == len(large) or group_rows + int(sizes[large[gi + 1]]) > p.roots_rows_per_run:
            _run_root_group(sess, sq8, gids, pts, offs_h, sizes, group, rows, p, sp, st, emit, consume, observer)
            group, group_rows = [], 0

    # small children one by one
    for c in small:
        a, b = int(offs_h[c]), int(offs_h[c + 1])
        cg = pts[a:b]
        ci = cg.long()
        sub = T.Sq8Matrix(sq8.codes[ci], sq8.scales[ci], sq8.norms[ci], sq8.dim)
        sess.upload_device(sub, cg)
        del sub, ci
        req = S.GpuSubtreePartitionRequest(point_ids=np.zeros(b - a, np.uint32), depth=1, parent_points=rows,
                                           min_recurse_size=p.min_recurse_size,
                                           memory_budget_bytes=p.gpu_workspace_budget_bytes or None)
        out = run_child(sess, req, sp)
        st["retries"] += 1 if out.retried else 0
        st["part_ms"] += out.partition_ms
        st["leaf_ms"] += out.leaf_ms
        st["runs"] += 1
        lay = T.LeafLayouts(out.leaf_row_ids[: out.leaf_rows], out.leaf_starts[: out.leaf_count],
                            out.leaf_sizes[: out.leaf_count].to(torch.int32),
                            out.leaf_starts[: out.leaf_count] * out.k, leaf_max, out.leaf_rows * out.k)
        rec, cnt, segs, nseg = emit(cg, lay, out.k, out.topk_ids, out.topk_dists)
        if observer is not None:
            observer(("child", c), cg, out, lay, rec, cnt, segs, nseg)
        consume(rec, cnt, segs, nseg)
        st["records"] += int(cnt)
        st["leaves"] += out.leaf_count
        st["leaf_rows"] += out.leaf_rows
        del rec, segs, out, lay
    if tl is not None:
        torch.cuda.synchronize()
        w_emit = time.perf_counter()
        targets, counts = tl.finish()
        tl_stats = dict(tl.stats, push_blocked_s=round(st["push_s"], 3), emit_done_s=round(w_emit - w1, 3))
        tl.close()
    else:
        targets, counts = hp.neighbors()
        torch.cuda.synchronize()
        hp.close()  # the reservoirs go before the image is packed (at 150M points they hold 96 GB)
    del sess
    prune_ms = 0.0
    if p.final_prune:
        torch.cuda.synchronize()
        q0 = time.perf_counter()
        targets, counts = G.robust_prune(points, targets, counts, p.l_max, p.prune_max_occlusion, p.prune_alpha,
                                         p.prune_saturate)
        torch.cuda.synchronize()
        prune_ms = (time.perf_counter() - q0) * 1e3
    image = G.pack_mem_index(targets, counts, start)
    torch.cuda.synchronize()
    w2 = time.perf_counter()
    stages = {"quantize_d0_ms": round((w1 - w0) * 1e3, 2), "d0_leaders": int(len(leader_rows)),
              "d0_fanout_top": p.fanout_top, "subtree_fanout_second": p.fanout_second,
              "children": len(children), "multi_root_children": len(large), "partition_runs": st["runs"],
              "children_and_pack_ms": round((w2 - w1) * 1e3, 2), "partition_ms": round(st["part_ms"], 2),
              "leaf_ms": round(st["leaf_ms"], 2), "leaves": st["leaves"], "leaf_rows": st["leaf_rows"],
              "edge_records": st["records"], "terminal_depth_retries": st["retries"],
              "emit_ms": round(st["emit_s"] * 1e3, 2), "reduce_ms": round(st["reduce_s"] * 1e3, 2),
              "final_prune_ms": round(prune_ms, 2)}
    if tl is not None:
        stages["tierlift"] = tl_stats
    if p.gpu_workspace_budget_bytes:
        # the largest task's workspace under the cap (a task above it fails its run)
        big = int(sizes.max())
        plan = S.plan_subtree(big, p.leaf_knn, min(p.max_leaders, D.GPU_QUEUE_LEADER_STRIDE), p.fanout_second,
                              p.gpu_workspace_budget_bytes, p.c_max)
        stages["largest_task_rows"] = big
        stages["largest_task_workspace_bytes"] = int(plan.required_bytes)
    return BuiltGraph(targets, counts, start, image, w2 - w0, stages)


@dataclass
class LeafChunk:
    """A batch of leaves of a many-root run as the observer sees it (the
    fields of a subtree run's output it reads)."""

    leaf_row_ids: torch.Tensor
    leaf_starts: torch.Tensor
    leaf_sizes: torch.Tensor
    leaf_count: int
    leaf_rows: int
    k: int
    topk_ids: torch.Tensor
    topk_dists: torch.Tensor


def _run_root_group(sess, sq8, gids, pts, offs_h, sizes, group, parent_points, p, sp, st, emit, consume, observer):
    """One many-root partition over the D0 children in ``group``, then the
    leaf top-k and record emission of its leaves in chunks."""
    dev = sq8.codes.device
    rows_t = torch.cat([pts[int(offs_h[c]):int(offs_h[c + 1])] for c in group])
    roffs = np.zeros(len(group) + 1, np.uint64)
    roffs[1:] = np.cumsum([int(sizes[c]) for c in group])
    seeds = np.array([S.subtree_root_seed(p.random_seed, 1, int(sizes[c]), parent_points, p.min_recurse_size)
                      for c in group], np.uint64)
    # the terminal-depth retry (rbc_partition.rs:15066-15115) run up front: a
    # root's tree under max(max_depth + 1, 1024) equals the first run's tree
    # when that one succeeds, and is the retry's tree when it fails; a root
    # would have failed iff one of its leaves lies deeper than max_depth
    md = max(p.max_depth + 1, TERMINAL_DEPTH_RECOVERY_FLOOR)
    ro = sess.partition_roots(sq8, rows_t, roffs, seeds, sp, depth=1, max_depth=md,
                              memory_budget_bytes=p.gpu_workspace_budget_bytes or None)
    st["runs"] += 1
    st["part_ms"] += ro.partition_ms
    lc = ro.leaf_count
    if lc == 0:
        return
    deepest = torch.zeros(len(group), dtype=torch.int32, device=dev)
    deepest.scatter_reduce_(0, ro.leaf_roots[:lc].long(), ro.leaf_depths[:lc], reduce="amax")
    st["retries"] += int((deepest > p.max_depth).sum().item())
    del rows_t, deepest
    starts = ro.leaf_starts[:lc].cpu().numpy()
    lsz = ro.leaf_sizes[:lc].cpu().numpy().astype(np.int64)
    k = p.leaf_knn
    leaf_max = max(256, p.c_max)
    ends = starts + lsz
    chunks = []
    l0 = 0
    while l0 < lc:
        # leaves [l0, l1) with at most leaf_chunk_rows rows (at least one leaf)
        l1 = int(np.searchsorted(ends, starts[l0] + p.leaf_chunk_rows, side="right"))
        l1 = max(l1, l0 + 1)
        chunks.append((l0, l1))
        l0 = l1
    # The leaf operator of chunk i + 1 is queued on its own stream before the
    # host waits for chunk i's record emission and merge (both synchronise the
    # caller's stream), so the GPU is not left idle while the host works.
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)  # default priority

    def launch(l0, l1):
        r0, r1 = int(starts[l0]), int(ends[l1 - 1])
        off = ro.leaf_starts[l0:l1]
        lay = T.LeafLayouts(ro.leaf_rows, off, ro.leaf_sizes[l0:l1], (off - r0) * k, leaf_max, (r1 - r0) * k)
        side.wait_stream(main)  # the layout tensors above were made on the caller's stream
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(side):
            e0.record(side)
            ids, d, ctr = T.leaf_topk(sq8, gids, lay, k, executor=sp.executor, stream=side)
            e1.record(side)
        return l0, l1, r0, r1, off, lay, ids, d, ctr, e0, e1

    def finish(job):
        l0, l1, r0, r1, off, lay, ids, d, ctr, e0, e1 = job
        main.wait_event(e1)
        for t in (ids, d, ctr):
            t.record_stream(main)  # used on the caller's stream from here on
        T.raise_on_overflow(ctr, "leaf top-k")
        st["leaf_ms"] += e0.elapsed_time(e1)
        q0 = time.perf_counter()
        rec, cnt, segs, nseg = emit(gids, lay, k, ids, d)
        q1 = time.perf_counter()
        if observer is not None:
            chunk = LeafChunk(ro.leaf_rows[r0:r1], off - r0, ro.leaf_sizes[l0:l1], l1 - l0, r1 - r0, k, ids, d)
            observer(("roots", st["runs"] - 1, l0), None, chunk, lay, rec, cnt, segs, nseg)
            del chunk
        q2 = time.perf_counter()
        consume(rec, cnt, segs, nseg)
        st["emit_s"] += q1 - q0
        st["reduce_s"] += time.perf_counter() - q2
        st["records"] += int(cnt)
        st["leaves"] += l1 - l0
        st["leaf_rows"] += r1 - r0

    pending = None
    for l0, l1 in chunks:
        job = launch(l0, l1)
        if pending is not None:
            finish(pending)
        pending = job
        del job
    if pending is not None:
        finish(pending)
    main.wait_stream(side)

