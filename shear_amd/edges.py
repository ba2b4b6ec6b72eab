"""Candidate records -> HashPrune edge records, on the GPU.

Host mirror of SHEAR's record-to-edge conversion (paths relative to
shear-core/src/algorithm/pipnn/):

* ``flush_compact_topk_batch_into_edges``  leaf_build.rs:1679-1829 -- every
  valid slot (j, d) of member row i becomes (i -> j, compute_hash(s_i, s_j), d)
  then (j -> i, compute_hash(s_j, s_i), d)
* ``compute_hash``                         hash_prune.rs:2239-2251
* ``EDGE_RECORD_DTYPE``                    SpillRecord16, spill_hashprune.rs:137-145

The conversion runs in libtessa_hip.so (``tessa_emit_edge_records``); this
module only moves buffers.  HashPrune evidence annotation and compact lune
pruning (reference options, off by default) are not offered: every record's
``flags`` is 0.
"""
from __future__ import annotations

import ctypes as C
import re
from typing import Sequence

import numpy as np
import torch

from . import _native as N
from .tessa import EMPTY_ID, CompactTopKBatch, LeafLayouts, _ptr, _stream_ptr

EDGE_RECORD_DTYPE = np.dtype([("src", "<u4"), ("dst", "<u4"), ("hash", "<u2"), ("flags", "<u2"), ("dist", "<f4")])
DEFAULT_M_HASH_BITS = 12  # params.rs:3345


def emit_edge_records(global_ids: torch.Tensor, layouts: LeafLayouts, k: int, topk_ids: torch.Tensor,
                      topk_dists: torch.Tensor, sketches: torch.Tensor, m_hash_bits: int = DEFAULT_M_HASH_BITS,
                      out: torch.Tensor | None = None, leaf_record_offsets: torch.Tensor | None = None,
                      stream: torch.cuda.Stream | None = None):
    """Edge records of every leaf of a leaf-top-k output, in the reference's order.

    ``global_ids`` (int32 view of u32, per resident row), ``topk_ids`` /
    ``topk_dists`` as written by ``tessa.leaf_topk`` with stride ``k``,
    ``sketches`` a [sketch_rows, width] f32 device tensor indexed by global id.
    Returns ``(records, count)``: ``records`` is the int32 [capacity, 4] buffer
    whose first ``count`` rows are 16-byte SpillRecord16 records.
    Synchronises the stream."""
    dev = topk_ids.device
    if sketches.dtype != torch.float32 or sketches.dim() != 2:
        raise ValueError("sketches must be a 2-D float32 tensor")
    if out is None:
        out = torch.empty((max(2 * layouts.output_len, 1), 4), dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or out.dim() != 2 or out.shape[1] != 4:
        raise ValueError("out must be an int32 [capacity, 4] tensor")
    if leaf_record_offsets is not None and (leaf_record_offsets.dtype != torch.int64
                                            or leaf_record_offsets.numel() < layouts.leaf_count + 1):
        raise ValueError("leaf_record_offsets must be int64 with leaf_count + 1 entries")
    lb = N.LeafBatch(_ptr(layouts.members), _ptr(layouts.member_offsets), _ptr(layouts.member_counts),
                     _ptr(layouts.output_offsets), layouts.leaf_count, layouts.max_leaf_rows, k, N.EXEC_MFMA, 0, 0)
    sk = N.SketchView(_ptr(sketches), sketches.shape[0], sketches.shape[1], m_hash_bits)
    count = C.c_uint64(0)
    N.check(N.load().tessa_emit_edge_records(_ptr(global_ids), global_ids.numel(), C.byref(lb), _ptr(topk_ids),
                                             _ptr(topk_dists), C.byref(sk), _ptr(out), out.shape[0],
                                             _ptr(leaf_record_offsets), C.byref(count), _stream_ptr(stream)),
            "edge records")
    return out, int(count.value)


def emit_edge_segments(global_ids: torch.Tensor, layouts: LeafLayouts, k: int, topk_ids: torch.Tensor,
                       topk_dists: torch.Tensor, sketches: torch.Tensor, m_hash_bits: int = DEFAULT_M_HASH_BITS,
                       out: torch.Tensor | None = None, segments: torch.Tensor | None = None,
                       stream: torch.cuda.Stream | None = None, unique: bool = False):
    """The records of ``emit_edge_records`` in source-grouped order with one
    segment per member row (tessa_emit_edge_segments).  Returns ``(records,
    count, segments, segment_count)``; ``segments`` is an int32 [capacity, 4]
    tensor of {src, first record lo, hi, count}.  Synchronises the stream.

    ``unique`` (tessa_emit_edge_segments_unique) leaves out the reverse
    record of each slot whose target row lists the source at the same
    distance: that row's forward record is the same record, so the set of
    records, and any HashPrune reduction of them, is unchanged; ``count`` is
    then the records written, with no gaps."""
    dev = topk_ids.device
    if out is None:
        out = torch.empty((max(2 * layouts.output_len, 1), 4), dtype=torch.int32, device=dev)
    if segments is None:
        segments = torch.empty((max(layouts.output_len // max(k, 1), layouts.leaf_count, 1), 4), dtype=torch.int32,
                               device=dev)
    if out.dtype != torch.int32 or out.dim() != 2 or out.shape[1] != 4:
        raise ValueError("out must be an int32 [capacity, 4] tensor")
    if segments.dtype != torch.int32 or segments.dim() != 2 or segments.shape[1] != 4:
        raise ValueError("segments must be an int32 [capacity, 4] tensor")
    lb = N.LeafBatch(_ptr(layouts.members), _ptr(layouts.member_offsets), _ptr(layouts.member_counts),
                     _ptr(layouts.output_offsets), layouts.leaf_count, layouts.max_leaf_rows, k, N.EXEC_MFMA, 0, 0)
    sk = N.SketchView(_ptr(sketches), sketches.shape[0], sketches.shape[1], m_hash_bits)
    count, nseg = C.c_uint64(0), C.c_uint64(0)
    fn = N.load().tessa_emit_edge_segments_unique if unique else N.load().tessa_emit_edge_segments
    N.check(fn(_ptr(global_ids), global_ids.numel(), C.byref(lb), _ptr(topk_ids), _ptr(topk_dists), C.byref(sk),
               _ptr(out), out.shape[0], _ptr(segments), segments.shape[0], C.byref(count), C.byref(nseg),
               _stream_ptr(stream)), "edge segments")
    return out, int(count.value), segments, int(nseg.value)


def records_to_numpy(records: torch.Tensor, count: int) -> np.ndarray:
    """First ``count`` records of an int32 [*, 4] record buffer as EDGE_RECORD_DTYPE."""
    raw = records[:count].contiguous().cpu().numpy()
    return raw.view(np.uint8).reshape(-1).view(EDGE_RECORD_DTYPE)


def flush_compact_topk_batches(batches: Sequence[CompactTopKBatch], sketches: np.ndarray,
                               m_hash_bits: int = DEFAULT_M_HASH_BITS, device="cuda") -> np.ndarray:
    """flush_compact_topk_batches (leaf_build.rs:1636-1678) up to the edge sink:
    the concatenated records of ``batches`` (host arrays), computed on the GPU.

    The batches are laid out as leaves of one upload (row stride = largest
    batch k, padded with empty slots).  A batch whose k exceeds rows - 1 is
    accepted when its slots beyond rank rows - 2 are empty (always the case
    for batches built by ``compact_batches_from_slices``)."""
    batches = [b for b in batches if b.rows > 0 and b.k > 0]  # leaf_build.rs:1695-1698
    if not batches:
        return np.zeros(0, EDGE_RECORD_DTYPE)
    stride = max(b.k for b in batches)
    for b in batches:
        if len(b.point_ids) != b.rows or len(b.topk_ids) != b.rows * b.k or len(b.topk_dists) != b.rows * b.k:
            raise ValueError(f"Invalid compact top-k batch shape: rows={b.rows} k={b.k} "
                             f"point_ids={len(b.point_ids)} topk_ids={len(b.topk_ids)} "
                             f"topk_dists={len(b.topk_dists)}")
        if b.k > max(b.rows - 1, 0):
            tail = np.asarray(b.topk_ids, np.uint32).reshape(b.rows, b.k)[:, max(b.rows - 1, 0):]
            if np.any(tail != EMPTY_ID):
                raise ValueError(f"batch {b.leaf_id}: k={b.k} > rows-1 with filled slots past rank rows-2")
    counts = np.array([b.rows for b in batches], np.int64)
    gids = np.concatenate([np.asarray(b.point_ids, np.uint32) for b in batches])
    ids = np.full((int(counts.sum()), stride), EMPTY_ID, np.uint32)
    dists = np.full((int(counts.sum()), stride), np.inf, np.float32)
    row = 0
    for b in batches:
        ids[row:row + b.rows, :b.k] = np.asarray(b.topk_ids, np.uint32).reshape(b.rows, b.k)
        dists[row:row + b.rows, :b.k] = np.asarray(b.topk_dists, np.float32).reshape(b.rows, b.k)
        row += b.rows
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64)
    lay = LeafLayouts.from_host(np.arange(len(gids), dtype=np.uint32), offs, counts, stride, device=device)
    g = torch.from_numpy(gids.view(np.int32)).to(device)
    t_ids = torch.from_numpy(ids.reshape(-1).view(np.int32)).to(device)
    t_d = torch.from_numpy(dists.reshape(-1)).to(device)
    sk = torch.from_numpy(np.ascontiguousarray(sketches, np.float32)).to(device)
    try:
        rec, n = emit_edge_records(g, lay, stride, t_ids, t_d, sk, m_hash_bits)
    except N.TessaError as e:
        # the device numbers leaves by upload position; name the batch's leaf_id
        m = re.search(r"outside leaf (\d+)", e.message)
        if m:
            leaf_id = batches[int(m.group(1))].leaf_id
            e.message = e.message[: m.start(1)] + str(leaf_id) + e.message[m.end(1):]
            e.args = (f"edge records: code={e.code} {e.message}",)
        raise
    return records_to_numpy(rec, n)
