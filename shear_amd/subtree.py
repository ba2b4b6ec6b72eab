"""Resident-subtree operator: recursive partition + leaf top-k over the HIP C ABI.

Mirrors (paths relative to shear-core/src/algorithm/pipnn/ in the reference):

* ``PiPNNSubtreeParams``          the PiPNNParams fields the path reads
                                  (params.rs:3362-3372 defaults)
* ``GpuSubtreePartitionRequest``  compute_backend.rs:1818-1826
* ``plan_subtree``                plan_gpu_persistent_subtree :1309-1488
* ``subtree_root_seed``           gpu_queue_root_seed :1597-1603
* ``SubtreeSession.process_quantized_subtree_l2_compact_topk``
                                  PiPNNComputeBackend::process_quantized_subtree_l2_compact_topk
                                  :3794-3805 -> GpuSubtreeTopKResult :1945-1951,
                                  batches from compact_batches_from_persistent_slices
                                  :32243-32339

All work runs in libtessa_hip.so; torch tensors only hold device memory.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native as N
from .tessa import CompactTopKBatch, compact_batches_from_slices

GPU_QUEUE_LEADER_STRIDE = 128  # compute_backend.rs:371


@dataclass
class PiPNNSubtreeParams:
    leaf_knn: int = 2
    c_min: int = 256
    c_max: int = 2048
    psamp_fraction: float = 0.001
    max_leaders: int = 1000
    max_depth: int = 10
    fanout_second: int = 3
    random_seed: int = 42
    gpu_workspace_budget_bytes: int = 0  # 0 = unlimited
    executor: int = N.EXEC_MFMA


@dataclass
class GpuSubtreePartitionRequest:
    point_ids: np.ndarray                 # u32 global ids of the resident rows
    root_leader_ids: np.ndarray | None = None  # resident row ids
    depth: int = 0
    parent_points: int = 0
    adaptive_c_max: int = 0
    min_recurse_size: int = 0
    memory_budget_bytes: int | None = None


@dataclass
class GpuSubtreeTopKResult:
    compact_batches: list[CompactTopKBatch]
    assignment_passes: int
    leaf_count: int
    max_active_points: int
    profile: dict = field(default_factory=dict)


def subtree_root_seed(random_seed: int, depth: int, point_count: int, parent_points: int,
                      min_recurse_size: int) -> int:
    return int(N.load().tessa_subtree_root_seed(random_seed & (2**64 - 1), depth, point_count, parent_points,
                                                min_recurse_size))


def plan_subtree(resident_rows: int, leaf_knn: int, max_leaders_per_node: int, max_fanout: int,
                 budget_bytes: int | None, c_max: int) -> N.SubtreePlan:
    plan = N.SubtreePlan()
    N.check(N.load().tessa_plan_subtree(resident_rows, leaf_knn, max_leaders_per_node, max_fanout,
                                        budget_bytes or 0, c_max, C.byref(plan)), "tessa_plan_subtree")
    return plan


@dataclass
class SubtreeDeviceOutput:
    """Device-resident result of one run (before any host copy)."""

    leaf_row_ids: torch.Tensor  # int32 view of u32
    leaf_starts: torch.Tensor   # int64
    leaf_sizes: torch.Tensor    # int64
    topk_ids: torch.Tensor      # int32 view of u32
    topk_dists: torch.Tensor    # f32
    counters: np.ndarray        # u64[159], reference layout
    leaf_counters: np.ndarray   # u64[32]
    leaf_count: int
    leaf_rows: int
    k: int
    levels: int
    partition_ms: float
    leaf_ms: float


@dataclass
class RootsDeviceOutput:
    """Leaves of a many-root partition (device tensors; member rows are SQ8 row ids)."""

    leaf_rows: torch.Tensor    # int32 view of u32 SQ8 rows, [>= leaf_rows_total]
    leaf_starts: torch.Tensor  # int64 [>= leaf_count]
    leaf_sizes: torch.Tensor   # int32 [>= leaf_count]
    leaf_roots: torch.Tensor   # int32 [>= leaf_count]: root index of each leaf
    leaf_depths: torch.Tensor  # int32 [>= leaf_count]
    leaf_count: int
    leaf_rows_total: int
    levels: int
    partition_ms: float
    counters: np.ndarray


class SubtreeSession:
    """One device, one stream, one uploaded resident subtree (the reference's
    CudaComputeBackend with its resident subtree workspace)."""

    def __init__(self, device: int = 0):
        self._lib = N.load()
        h = C.c_void_p()
        N.check(self._lib.tessa_session_create(C.byref(N.TessaConfig(device, 0)), C.byref(h)), "session create")
        self._h = h
        self.device = device
        self.rows = 0
        self._keep = ()

    def close(self):
        if self._h:
            N.check(self._lib.tessa_session_destroy(self._h), "session destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, codes: np.ndarray, scales: np.ndarray, norms: np.ndarray, global_ids: np.ndarray, dim: int):
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        norms = np.ascontiguousarray(norms, np.float32)
        gids = np.ascontiguousarray(global_ids, np.uint32)
        view = N.Sq8View(codes.ctypes.data, scales.ctypes.data, norms.ctypes.data, gids.ctypes.data,
                         codes.shape[0], dim, codes.shape[1])
        N.check(self._lib.tessa_session_upload_sq8(self._h, C.byref(view)), "session upload")
        self.rows = codes.shape[0]
        self.global_ids = gids

    def _request(self, rows: int, request: GpuSubtreePartitionRequest, params: PiPNNSubtreeParams,
                 partition_only: bool):
        """-> (tessa_subtree_request, plan, k, root leader array kept alive by the caller)."""
        famp = max(params.fanout_second, 1)
        max_leaders = min(max(params.max_leaders, 1), GPU_QUEUE_LEADER_STRIDE)
        plan = plan_subtree(rows, params.leaf_knn, max_leaders, famp, request.memory_budget_bytes,
                            params.c_max)
        if not plan.supported:
            raise N.TessaError(_status(4, plan.overflow_flags,
                                       f"CUDA persistent strict error: unsupported subtree "
                                       f"fallback_reason_flags=0x{plan.fallback_reason_flags:x}"), "plan")
        seed = subtree_root_seed(params.random_seed, request.depth, len(request.point_ids),
                                 request.parent_points, request.min_recurse_size)
        k = 0 if partition_only else min(params.leaf_knn, max(rows - 1, 0))
        roots = (np.zeros(0, np.uint32) if request.root_leader_ids is None
                 else np.ascontiguousarray(request.root_leader_ids, np.uint32))
        rq = N.SubtreeRequest(
            roots.ctypes.data if len(roots) else None, len(roots), request.depth, seed,
            max(params.leaf_knn, 1), famp, params.max_depth, max_leaders, plan.leaf_min, plan.leaf_max,
            plan.small_node_limit, np.float32(params.psamp_fraction).item(), params.executor,
            1 if partition_only else 0, plan.max_leaf_count, plan.max_leaf_rows)
        return rq, plan, k, roots

    def submit_owned_quantized_subtree_l2_compact_topk(
            self, request: GpuSubtreePartitionRequest, codes: np.ndarray, scales: np.ndarray, norms: np.ndarray,
            global_ids: np.ndarray, dim: int, params: PiPNNSubtreeParams) -> "DeferredGpuSubtreeTopK":
        """compute_backend.rs:3807-3815: queue one task (its own SQ8 rows) on the
        session's worker; returns at once.  ``finish()`` of the result waits for
        the device work and the D2H into a pinned slot, builds the compact
        batches and releases the slot (CudaDeferredPinnedQuantizedScatter,
        compute_backend.rs:31432-31497)."""
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        norms = np.ascontiguousarray(norms, np.float32)
        gids = np.ascontiguousarray(global_ids, np.uint32)
        view = N.Sq8View(codes.ctypes.data, scales.ctypes.data, norms.ctypes.data, gids.ctypes.data,
                         codes.shape[0], dim, codes.shape[1])
        rq, plan, k, roots = self._request(codes.shape[0], request, params, False)
        seq = C.c_uint64(0)
        N.check(self._lib.tessa_session_submit_subtree(self._h, C.byref(view), C.byref(rq), C.byref(seq)),
                "tessa_session_submit_subtree")
        self.rows = codes.shape[0]
        self.global_ids = gids
        owned = (codes, scales, norms, gids, roots)  # the job reads these until it is waited for
        est = int(plan.max_leaf_rows) * (4 + k * 8) + int(plan.max_leaf_count) * 16
        return DeferredGpuSubtreeTopK(est, _PinnedScatter(self, int(seq.value), gids, params, owned))

    def set_assignment_capture(self, min_members: int = 256) -> None:
        """Record the assignment passes of nodes with >= min_members rows in
        each following run (0: off); the partition side of the TESSA capture
        (compute_backend.rs:5415-5546)."""
        N.check(self._lib.tessa_session_set_assignment_capture(self._h, min_members), "assignment capture")

    def captured_assignments(self) -> list[dict]:
        """The last run's captured passes in pass order: depth, retry, r_h,
        padded_dim, member_ids and leader_ids (global ids)."""
        nt, ni = C.c_uint64(0), C.c_uint64(0)
        N.check(self._lib.tessa_session_captured_assignments(self._h, None, 0, None, 0, C.byref(nt), C.byref(ni)),
                "captured assignments")
        tasks = (N.CapturedAssignment * max(nt.value, 1))()
        ids = np.zeros(max(ni.value, 1), np.uint32)
        N.check(self._lib.tessa_session_captured_assignments(self._h, tasks, nt.value, ids.ctypes.data, ni.value,
                                                             C.byref(nt), C.byref(ni)), "captured assignments")
        out = []
        for t in tasks[: nt.value]:
            out.append({"depth": t.depth, "retry": t.retry, "r_h": t.r_h, "padded_dim": t.padded_dim,
                        "member_ids": ids[t.member_offset: t.member_offset + t.member_count].copy(),
                        "leader_ids": ids[t.leader_offset: t.leader_offset + t.leader_count].copy()})
        return out

    def upload_device(self, sq8, global_ids: torch.Tensor):
        """Resident set from device tensors (an Sq8Matrix and int32-viewed u32
        global ids): a device-to-device copy into the session."""
        view = sq8.view(global_ids)
        # the session copies on its own stream: the tensors' producers on
        # torch's current stream must have finished
        torch.cuda.current_stream(sq8.codes.device).synchronize()
        N.check(self._lib.tessa_session_upload_sq8(self._h, C.byref(view)), "session upload")
        self.rows = sq8.rows
        self.global_ids = None

    def run(self, request: GpuSubtreePartitionRequest, params: PiPNNSubtreeParams,
            partition_only: bool = False) -> SubtreeDeviceOutput:
        rq, plan, k, roots = self._request(self.rows, request, params, partition_only)
        dev = torch.device("cuda", self.device)
        max_rows = max(int(plan.max_leaf_rows), 1)
        max_leaves = max(int(plan.max_leaf_count), 1)
        out_rows = torch.empty(max_rows, dtype=torch.int32, device=dev)
        out_starts = torch.empty(max_leaves, dtype=torch.int64, device=dev)
        out_sizes = torch.empty(max_leaves, dtype=torch.int64, device=dev)
        out_ids = torch.empty(max(max_rows * k, 1), dtype=torch.int32, device=dev)
        out_d = torch.empty(max(max_rows * k, 1), dtype=torch.float32, device=dev)
        counters = np.zeros(N.SUBTREE_COUNTER_WORDS, np.uint64)
        leaf_counters = np.zeros(N.COUNTER_WORDS, np.uint64)
        out = N.SubtreeOutput(out_rows.data_ptr(), out_starts.data_ptr(), out_sizes.data_ptr(),
                              out_ids.data_ptr(), out_d.data_ptr(), counters.ctypes.data,
                              leaf_counters.ctypes.data, 0, 0, 0, 0, 0.0, 0.0)
        torch.cuda.synchronize(dev)  # outputs allocated on torch's stream
        st = self._lib.tessa_session_run_subtree(self._h, C.byref(rq), C.byref(out))
        N.check(st, "tessa_session_run_subtree")
        return SubtreeDeviceOutput(out_rows, out_starts, out_sizes, out_ids, out_d, counters, leaf_counters,
                                   int(out.leaf_count), int(out.leaf_rows), int(out.k), int(out.levels),
                                   float(out.partition_ms), float(out.leaf_ms))

    def partition_roots(self, sq8, rows: torch.Tensor, root_offsets: np.ndarray, root_seeds: np.ndarray,
                        params: PiPNNSubtreeParams, depth: int = 1, max_depth: int | None = None,
                        memory_budget_bytes: int | None = None) -> RootsDeviceOutput:
        """Partition many subtree roots in one run (tessa_session_partition_roots):
        root i owns the SQ8 rows rows[root_offsets[i]:root_offsets[i+1]]
        (``rows`` a device int32 view of u32 row ids into ``sq8``, ascending per
        root) and starts from root_seeds[i] at ``depth``.  Each root is planned
        as a task of its own (``plan_subtree`` under ``memory_budget_bytes``);
        every root must be a large one (more than leaf_max rows or a fanout
        probe beyond the small-node scratch)."""
        offs = np.ascontiguousarray(root_offsets, np.uint64)
        seeds = np.ascontiguousarray(root_seeds, np.uint64)
        famp = max(params.fanout_second, 1)
        max_leaders = min(max(params.max_leaders, 1), GPU_QUEUE_LEADER_STRIDE)
        leaf_cap = row_cap = 0
        first = None
        for n in np.diff(offs.astype(np.int64)).tolist():
            plan = plan_subtree(int(n), params.leaf_knn, max_leaders, famp, memory_budget_bytes, params.c_max)
            if not plan.supported:
                raise N.TessaError(_status(4, plan.overflow_flags,
                                           f"CUDA persistent strict error: unsupported subtree "
                                           f"fallback_reason_flags=0x{plan.fallback_reason_flags:x}"), "plan")
            key = (plan.leaf_min, plan.leaf_max, plan.small_node_limit)
            if first is None:
                first = key
            elif key != first:
                raise ValueError(f"roots planned with different leaf bounds {key} != {first}")
            leaf_cap += int(plan.max_leaf_count)
            row_cap += int(plan.max_leaf_rows)
        dev = torch.device("cuda", self.device)
        out_rows = torch.empty(max(row_cap, 1), dtype=torch.int32, device=dev)
        out_starts = torch.empty(max(leaf_cap, 1), dtype=torch.int64, device=dev)
        out_sizes = torch.empty(max(leaf_cap, 1), dtype=torch.int32, device=dev)
        out_roots = torch.empty(max(leaf_cap, 1), dtype=torch.int32, device=dev)
        out_depths = torch.empty(max(leaf_cap, 1), dtype=torch.int32, device=dev)
        counters = np.zeros(N.SUBTREE_COUNTER_WORDS, np.uint64)
        view = N.Sq8View(sq8.codes.data_ptr(), sq8.scales.data_ptr(), sq8.norms.data_ptr(), None, sq8.rows,
                         sq8.dim, sq8.padded_dim)
        rq = N.RootsRequest(rows.data_ptr(), offs.ctypes.data, seeds.ctypes.data, len(seeds), depth, famp,
                            max_depth if max_depth is not None else params.max_depth, max_leaders, first[0],
                            first[1], first[2], np.float32(params.psamp_fraction).item(), 0, leaf_cap, row_cap)
        out = N.RootsOutput(out_rows.data_ptr(), out_starts.data_ptr(), out_sizes.data_ptr(), out_roots.data_ptr(),
                            out_depths.data_ptr(), counters.ctypes.data, 0, 0, 0, 0.0)
        torch.cuda.synchronize(dev)  # inputs and outputs come from torch's stream
        N.check(self._lib.tessa_session_partition_roots(self._h, C.byref(view), C.byref(rq), C.byref(out)),
                "tessa_session_partition_roots")
        return RootsDeviceOutput(out_rows, out_starts, out_sizes, out_roots, out_depths, int(out.leaf_count),
                                 int(out.leaf_rows_total), int(out.levels), float(out.partition_ms), counters)

    def process_quantized_subtree_l2_compact_topk(self, request: GpuSubtreePartitionRequest,
                                                  params: PiPNNSubtreeParams) -> GpuSubtreeTopKResult:
        r = self.run(request, params)
        lc, lr = r.leaf_count, r.leaf_rows
        leaf_row_ids = r.leaf_row_ids[:lr].cpu().numpy().view(np.uint32)
        starts = r.leaf_starts[:lc].cpu().numpy().astype(np.int64)
        sizes = r.leaf_sizes[:lc].cpu().numpy().astype(np.int64)
        ids = r.topk_ids[: lr * r.k].cpu().numpy().view(np.uint32)
        d = r.topk_dists[: lr * r.k].cpu().numpy()
        batches = compact_batches_from_slices(np.asarray(request.point_ids, np.uint32), leaf_row_ids, starts,
                                              sizes, ids, d, r.k, params.leaf_knn)
        return GpuSubtreeTopKResult(
            compact_batches=batches,
            assignment_passes=int(r.counters[N.P_ASSIGNMENT_PASSES]),
            leaf_count=lc,
            max_active_points=int(r.counters[N.P_MAX_ACTIVE]),
            profile={"counters": r.counters, "leaf_counters": r.leaf_counters, "levels": r.levels,
                     "partition_ms": r.partition_ms, "leaf_ms": r.leaf_ms},
        )


class _PinnedScatter:
    """DeferredGpuSubtreeScatter of one submission (compute_backend.rs:1958-1960)."""

    def __init__(self, session: SubtreeSession, seq: int, global_ids: np.ndarray, params: PiPNNSubtreeParams,
                 owned):
        self._session, self._seq, self._gids, self._params, self._owned = session, seq, global_ids, params, owned

    def finish(self) -> GpuSubtreeTopKResult:
        lib, h = self._session._lib, self._session._h
        r = N.SubtreeHostResult()
        st = lib.tessa_session_wait(h, self._seq, C.byref(r))
        try:
            N.check(st, "tessa_session_wait")
            lc, lr, k = int(r.leaf_count), int(r.leaf_rows), int(r.k)

            def arr(ptr, n, ctype, dt):
                if n == 0:
                    return np.zeros(0, dt)
                return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), shape=(n,)).astype(dt, copy=True)

            rows = arr(r.leaf_row_ids, lr, C.c_uint32, np.uint32)
            starts = arr(r.leaf_starts, lc, C.c_uint64, np.int64)
            sizes = arr(r.leaf_sizes, lc, C.c_uint64, np.int64)
            ids = arr(r.topk_ids, lr * k, C.c_uint32, np.uint32)
            d = arr(r.topk_dists, lr * k, C.c_float, np.float32)
            counters = arr(r.counters, N.SUBTREE_COUNTER_WORDS, C.c_uint64, np.uint64)
            leaf_counters = arr(r.leaf_counters, N.COUNTER_WORDS, C.c_uint64, np.uint64)
        finally:
            lib.tessa_session_release(h, self._seq)
            self._owned = None
        batches = compact_batches_from_slices(self._gids, rows, starts, sizes, ids, d, k, self._params.leaf_knn)
        return GpuSubtreeTopKResult(
            compact_batches=batches,
            assignment_passes=int(counters[N.P_ASSIGNMENT_PASSES]),
            leaf_count=lc,
            max_active_points=int(counters[N.P_MAX_ACTIVE]),
            profile={"counters": counters, "leaf_counters": leaf_counters, "levels": int(r.levels),
                     "partition_ms": float(r.partition_ms), "leaf_ms": float(r.leaf_ms)},
        )


@dataclass
class DeferredGpuSubtreeTopK:
    """compute_backend.rs:1958-1961."""

    estimated_host_bytes: int
    scatter: _PinnedScatter

    def finish(self) -> GpuSubtreeTopKResult:
        return self.scatter.finish()


def _status(code: int, flags: int, msg: str) -> N.TessaStatus:
    s = N.TessaStatus()
    s.code = code
    s.overflow_flags = flags
    s.msg = msg.encode()[:511]
    return s
