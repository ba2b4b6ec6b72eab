"""Host-side mirror of SHEAR's TESSA operator interface over the HIP C ABI.

Names and argument meanings follow the reference (paths relative to
shear-core/src/algorithm/pipnn/):

* ``quantize_sq_int8_matrix``   dco_sq_int8.rs:1331-1375 (runs on the GPU here,
                                bit-identical to the reference CPU quantizer)
* ``TessaLeafLayout`` /
  ``TessaAssignmentLayout``     tessa_replay.rs:1031-1047
* ``leaf_topk``                 gpu_persistent_subtree_topk_only, leaf leg of
                                TessaCudaReplaySession::run_mode
                                (compute_backend.rs:16146-16334, :34841)
* ``assignment_replay``         gpu_tessa_assignment_replay (compute_backend.rs:15729)
* ``CompactTopKBatch`` /
  ``compact_batches_from_slices`` leaf_build.rs:271-282,
                                compute_backend.rs:32243-32339

Device tensors are torch tensors on ``cuda`` (allocation and stream plumbing
only); every computation happens in libtessa_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import _native as N

SQ_INT8_DEFAULT_K_ALIGN = 16  # dco_sq_int8.rs:14
SQ_INT8_DEFAULT_BITS = 8  # dco_sq_int8.rs:15
STABLE_DISTANCE_TIE_EPS = 2.0e-5  # mod.rs:74
EMPTY_ID = 0xFFFFFFFF
EMPTY_DIST = np.float32(3.4028234663852886e38)


def sq_int8_padded_dim(dim: int, k_align: int = SQ_INT8_DEFAULT_K_ALIGN) -> int:
    """dco_sq_int8.rs:1216-1224."""
    if dim <= 0:
        raise ValueError("SQ-int8 quantization requires dim > 0")
    k_align = max(k_align, 1)
    return -(-dim // k_align) * k_align


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def _stream_ptr(stream: torch.cuda.Stream | None) -> int | None:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None


@dataclass
class Sq8Matrix:
    """SqInt8Matrix (dco_sq_int8.rs) held in device memory."""

    codes: torch.Tensor  # int8 [rows, padded_dim]
    scales: torch.Tensor  # f32 [rows]
    norms: torch.Tensor  # f32 [rows]
    dim: int

    @property
    def rows(self) -> int:
        return int(self.codes.shape[0])

    @property
    def padded_dim(self) -> int:
        return int(self.codes.shape[1])

    def view(self, global_ids: torch.Tensor) -> N.Sq8View:
        if global_ids.dtype != torch.int32 or global_ids.numel() != self.rows:
            raise ValueError("global_ids must be int32 (u32 bits) with one entry per row")
        return N.Sq8View(_ptr(self.codes), _ptr(self.scales), _ptr(self.norms), _ptr(global_ids),
                         self.rows, self.dim, self.padded_dim)


def quantize_sq_int8_matrix(x: torch.Tensor, k_align: int = SQ_INT8_DEFAULT_K_ALIGN,
                            bits: int = SQ_INT8_DEFAULT_BITS,
                            stream: torch.cuda.Stream | None = None) -> Sq8Matrix:
    """Per-vector symmetric SQ8 of an f32 [rows, dim] device matrix.

    Raises ValueError on a non-finite value, as the reference does.
    """
    if x.dtype != torch.float32 or x.dim() != 2:
        raise ValueError("x must be a 2-D float32 tensor")
    x = x.contiguous()
    rows, dim = x.shape
    pd = sq_int8_padded_dim(dim, k_align)
    dev = x.device
    codes = torch.empty((rows, pd), dtype=torch.int8, device=dev)
    scales = torch.empty(rows, dtype=torch.float32, device=dev)
    norms = torch.empty(rows, dtype=torch.float32, device=dev)
    bad = torch.empty(1, dtype=torch.int64, device=dev)
    N.check(N.load().tessa_sq8_quantize(_ptr(x), rows, dim, pd, bits, _ptr(codes), _ptr(scales),
                                        _ptr(norms), _ptr(bad), _stream_ptr(stream)),
            "tessa_sq8_quantize")
    bad_row = int(bad.item()) & 0xFFFFFFFFFFFFFFFF
    if bad_row != 0xFFFFFFFFFFFFFFFF:
        raise ValueError(f"SQ-int8 cannot quantize non-finite value in row {bad_row}")
    return Sq8Matrix(codes, scales, norms, dim)


@dataclass
class LeafLayouts:
    """Device copy of TessaLeafLayout[] (tessa_replay.rs:1041-1047)."""

    members: torch.Tensor  # int32 (u32) local rows, concatenated
    member_offsets: torch.Tensor  # int64
    member_counts: torch.Tensor  # int32
    output_offsets: torch.Tensor  # int64
    max_leaf_rows: int
    output_len: int

    @property
    def leaf_count(self) -> int:
        return int(self.member_counts.numel())

    @staticmethod
    def from_host(members: np.ndarray, member_offsets: np.ndarray, member_counts: np.ndarray,
                  k: int, device="cuda") -> "LeafLayouts":
        counts = np.asarray(member_counts, dtype=np.int64)
        out_off = np.zeros(len(counts), dtype=np.int64)
        if len(counts) > 1:
            out_off[1:] = np.cumsum(counts[:-1] * k)
        return LeafLayouts(
            torch.from_numpy(np.asarray(members, dtype=np.uint32).view(np.int32)).to(device),
            torch.from_numpy(np.asarray(member_offsets, dtype=np.int64)).to(device),
            torch.from_numpy(counts.astype(np.uint32).view(np.int32)).to(device),
            torch.from_numpy(out_off).to(device),
            int(counts.max()) if len(counts) else 0,
            int((counts * k).sum()),
        )

    @staticmethod
    def contiguous(leaf_count: int, leaf_rows: int, k: int, device="cuda") -> "LeafLayouts":
        """Leaves of `leaf_rows` consecutive resident rows (the leaf microbench)."""
        members = torch.arange(leaf_count * leaf_rows, dtype=torch.int32, device=device)
        offs = torch.arange(leaf_count, dtype=torch.int64, device=device) * leaf_rows
        counts = torch.full((leaf_count,), leaf_rows, dtype=torch.int32, device=device)
        return LeafLayouts(members, offs, counts, offs * k, leaf_rows, leaf_count * leaf_rows * k)


def leaf_topk(sq8: Sq8Matrix, global_ids: torch.Tensor, layouts: LeafLayouts, k: int,
              executor: int = N.EXEC_MFMA, out_ids: torch.Tensor | None = None,
              out_dists: torch.Tensor | None = None, counters: torch.Tensor | None = None,
              stream: torch.cuda.Stream | None = None, debug_rerun_every: int = 0,
              phase_ms: list | None = None, no_alloc: bool = False):
    """Enqueue the leaf operator; returns (ids int32 view of u32, dists f32, counters int64).

    With ``phase_ms`` (a list) the call synchronises and appends the hipEvent
    times of its kernels in ms: MFMA filter, select (each summed over the
    call's batches), chain replay, exact re-run.  ``no_alloc`` calls the entry
    point that keeps its scratch in a static device array (at most 65,536
    member rows per call; ``phase_ms`` is ignored then)."""
    dev = sq8.codes.device
    if out_ids is None:
        out_ids = torch.empty(layouts.output_len, dtype=torch.int32, device=dev)
    if out_dists is None:
        out_dists = torch.empty(layouts.output_len, dtype=torch.float32, device=dev)
    if counters is None:
        counters = torch.zeros(N.COUNTER_WORDS, dtype=torch.int64, device=dev)
    view = sq8.view(global_ids)
    lb = N.LeafBatch(_ptr(layouts.members), _ptr(layouts.member_offsets), _ptr(layouts.member_counts),
                     _ptr(layouts.output_offsets), layouts.leaf_count, layouts.max_leaf_rows, k, executor,
                     debug_rerun_every, 0)
    if no_alloc:
        N.check(N.load().tessa_leaf_topk_noalloc(C.byref(view), C.byref(lb), _ptr(out_ids), _ptr(out_dists),
                                                 _ptr(counters), _stream_ptr(stream)), "tessa_leaf_topk_noalloc")
    elif phase_ms is None:
        N.check(N.load().tessa_leaf_topk(C.byref(view), C.byref(lb), _ptr(out_ids), _ptr(out_dists),
                                         _ptr(counters), _stream_ptr(stream)), "tessa_leaf_topk")
    else:
        ph = (C.c_float * 5)()
        N.check(N.load().tessa_leaf_topk_profiled(C.byref(view), C.byref(lb), _ptr(out_ids), _ptr(out_dists),
                                                  _ptr(counters), _stream_ptr(stream), ph),
                "tessa_leaf_topk_profiled")
        phase_ms.append([float(ph[i]) for i in range(5)])
    return out_ids, out_dists, counters


@dataclass
class AssignLayouts:
    """Device copy of TessaAssignmentLayout[] (tessa_replay.rs:1031-1039)."""

    members: torch.Tensor
    leaders: torch.Tensor
    member_offsets: torch.Tensor
    member_counts: torch.Tensor
    leader_offsets: torch.Tensor
    leader_counts: torch.Tensor
    r_h: torch.Tensor
    output_offsets: torch.Tensor
    max_members: int
    output_len: int

    @property
    def task_count(self) -> int:
        return int(self.member_counts.numel())

    @staticmethod
    def from_host(members, leaders, member_offsets, member_counts, leader_offsets, leader_counts, r_h,
                  device="cuda") -> "AssignLayouts":
        mc = np.asarray(member_counts, dtype=np.int64)
        rh = np.asarray(r_h, dtype=np.int64)
        lc = np.asarray(leader_counts, dtype=np.int64)
        if np.any(rh < 1) or np.any(rh > 4) or np.any(lc < rh) or np.any(lc > 128):
            raise ValueError("each task needs 1 <= r_h <= 4, r_h <= leaders <= 128")
        out_off = np.zeros(len(mc), dtype=np.int64)
        if len(mc) > 1:
            out_off[1:] = np.cumsum(mc[:-1] * rh[:-1])
        u32 = lambda a: torch.from_numpy(np.asarray(a, dtype=np.uint32).view(np.int32)).to(device)  # noqa: E731
        return AssignLayouts(u32(members), u32(leaders), u32(member_offsets), u32(mc), u32(leader_offsets),
                             u32(lc), u32(rh), torch.from_numpy(out_off).to(device),
                             int(mc.max()) if len(mc) else 0, int((mc * rh).sum()))


def assignment_replay(sq8: Sq8Matrix, global_ids: torch.Tensor, layouts: AssignLayouts,
                      counters: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None):
    dev = sq8.codes.device
    out_ids = torch.empty(layouts.output_len, dtype=torch.int32, device=dev)
    out_dists = torch.empty(layouts.output_len, dtype=torch.float32, device=dev)
    if counters is None:
        counters = torch.zeros(N.COUNTER_WORDS, dtype=torch.int64, device=dev)
    view = sq8.view(global_ids)
    tb = N.AssignBatch(_ptr(layouts.members), _ptr(layouts.leaders), _ptr(layouts.member_offsets),
                       _ptr(layouts.member_counts), _ptr(layouts.leader_offsets), _ptr(layouts.leader_counts),
                       _ptr(layouts.r_h), _ptr(layouts.output_offsets), layouts.task_count, layouts.max_members)
    N.check(N.load().tessa_assign_replay(C.byref(view), C.byref(tb), _ptr(out_ids), _ptr(out_dists),
                                         _ptr(counters), _stream_ptr(stream)), "tessa_assign_replay")
    return out_ids, out_dists, counters


def raise_on_overflow(counters: torch.Tensor, what: str) -> None:
    """Host check of the device overflow word (after synchronising)."""
    flags = int(counters[N.C_OVERFLOW_FLAGS].item()) & 0xFFFFFFFFFFFFFFFF
    if flags:
        raise RuntimeError(f"HIP {what} overflow: overflow_flags=0x{flags:x} "
                           f"overflow_labels={N.overflow_labels(flags)}")


# ---- candidate records ----------------------------------------------------

@dataclass
class CompactTopKBatch:
    """leaf_build.rs:271-282."""

    leaf_id: int
    point_ids: np.ndarray  # u32 global ids in member order
    rows: int
    k: int
    topk_ids: np.ndarray  # u32 [rows*k], EMPTY_ID = none
    topk_dists: np.ndarray  # f32 [rows*k]
    estimated_dtoh_bytes: int = 0
    lune_witness_pivot_ranks: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    lune_witness_margins: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))


def compact_batches_from_slices(global_ids: np.ndarray, leaf_row_ids: np.ndarray, leaf_starts: np.ndarray,
                                leaf_sizes: np.ndarray, topk_ids: np.ndarray, topk_dists: np.ndarray,
                                max_k: int, leaf_knn: int) -> list[CompactTopKBatch]:
    """compute_backend.rs:32243-32339: one batch per leaf, k = min(leaf_knn, size-1),
    rows copied from the max_k-strided device slices."""
    rows_total = len(leaf_row_ids)
    batches = []
    for leaf, (start, size) in enumerate(zip(leaf_starts.tolist(), leaf_sizes.tolist())):
        end = start + size
        if end > rows_total:
            raise ValueError(f"persistent subtree leaf {leaf} end {end} exceeds rows {rows_total}")
        k = min(leaf_knn, max(size - 1, 0))
        local = leaf_row_ids[start:end]
        if np.any(local >= len(global_ids)):
            raise ValueError("leaf row outside resident global id table")
        src = (np.arange(start, end)[:, None] * max_k + np.arange(k)[None, :]).reshape(-1)
        batches.append(CompactTopKBatch(
            leaf_id=leaf,
            point_ids=np.asarray(global_ids)[local].astype(np.uint32),
            rows=size,
            k=k,
            topk_ids=np.asarray(topk_ids, dtype=np.uint32)[src] if k else np.zeros(0, np.uint32),
            topk_dists=np.asarray(topk_dists, dtype=np.float32)[src] if k else np.zeros(0, np.float32),
            estimated_dtoh_bytes=size * k * 8,
        ))
    return batches


def replay_leaf_blocks(member_counts: Sequence[int], k: int):
    """TessaCandidateBlock list for leaf tasks (tessa_replay.rs:1394-1399)."""
    from .replay import TessaCandidateBlock

    blocks, off = [], 0
    for n in member_counts:
        blocks.append(TessaCandidateBlock(off, int(n), k, int(n) * max(int(n) - 1, 0)))
        off += int(n) * k
    return blocks
