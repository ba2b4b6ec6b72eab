"""Graph emission and the recall harness: the `_mem.index` file of a
neighbour table, packed on the GPU, and greedy search over it.

Host mirror of DirectMemGraphWriter (shear-core/src/index/inmem_index/
pipnn_oom_writer.rs:23-72): ``write_mem_index`` writes what create +
write_node (per point, id order) + finish write; the byte image itself is
built by ``tessa_graph_pack`` in libtessa_hip.so.  ``read_mem_index`` parses
the same layout back (header: index_size u64, max_degree u32, start u32,
num_frozen_pts u64; rows: degree u32 then ids, little-endian).

``robust_prune`` is the final RobustPrune (final_prune_pipnn,
shear-core/src/index/inmem_index/pipnn_builder.rs:287-330, with
algorithm/prune/prune.rs:17-214) run by ``tessa_robust_prune``.
``greedy_search`` is InmemIndex::search (shear-core/src/index/inmem_index/
inmem_index.rs:523-590, greedy_search algorithm/search/search.rs:137-233) run
by ``tessa_graph_search``, one wavefront per query; ``recall_at_k`` is the
search app's recall (apps/search_shear_index/src/main.rs:388-413).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import torch

from . import _native as N
from .tessa import _ptr, _stream_ptr


def pack_mem_index(targets: torch.Tensor, counts: torch.Tensor, start: int, num_frozen: int = 0,
                   stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """Device uint8 tensor holding the file image.  ``targets`` int32
    [num_points, row_stride] (row p's ids first), ``counts`` int32 [num_points]."""
    if targets.dim() != 2 or targets.dtype != torch.int32 or counts.dtype != torch.int32:
        raise ValueError("targets must be int32 [num_points, row_stride] and counts int32 [num_points]")
    n, stride = targets.shape
    if counts.numel() != n:
        raise ValueError(f"counts has {counts.numel()} entries for {n} rows")
    t = targets.contiguous()
    size = C.c_uint64(0)
    lib = N.load()
    N.check(lib.tessa_graph_pack(_ptr(t), _ptr(counts), n, stride, start, num_frozen, None, 0, C.byref(size),
                                 _stream_ptr(stream)), "graph pack")
    out = torch.empty((size.value + 7) // 8, dtype=torch.int64, device=t.device)  # 8-byte aligned
    N.check(lib.tessa_graph_pack(_ptr(t), _ptr(counts), n, stride, start, num_frozen, _ptr(out), out.numel() * 8,
                                 C.byref(size), _stream_ptr(stream)), "graph pack")
    return out.view(torch.uint8)[: size.value]


def write_mem_index(path, targets: torch.Tensor, counts: torch.Tensor, start: int, num_frozen: int = 0) -> int:
    """Write the `_mem.index` file; returns its size in bytes."""
    img = pack_mem_index(targets, counts, start, num_frozen)
    data = img.cpu().numpy()
    Path(path).write_bytes(data.tobytes())
    return len(data)


def read_mem_index(src):
    """(start, num_frozen, max_degree, rows) from a path or bytes; rows is a
    list of uint32 arrays in point order."""
    buf = Path(src).read_bytes() if not isinstance(src, (bytes, bytearray, memoryview)) else bytes(src)
    size, max_degree, start, frozen = np.frombuffer(buf[:24], dtype=np.dtype("<u8,<u4,<u4,<u8"))[0]
    if size != len(buf):
        raise ValueError(f"index_size {size} != {len(buf)} bytes")
    words = np.frombuffer(buf[24:], dtype="<u4")
    rows, i = [], 0
    while i < len(words):
        d = int(words[i])
        rows.append(words[i + 1: i + 1 + d].copy())
        i += 1 + d
    if i != len(words):
        raise ValueError("truncated row")
    return int(start), int(frozen), int(max_degree), rows


def greedy_search(data: torch.Tensor, targets: torch.Tensor, counts: torch.Tensor, start: int,
                  queries: torch.Tensor, L: int, K: int, stream: torch.cuda.Stream | None = None):
    """(ids int32 [q, K] (-1 past the list), squared-L2 f32 [q, K], distance
    evaluations int32 [q]) of the greedy search from ``start`` with list size L.
    ``data`` f32 [n, dim], ``targets`` int32 [n, row_stride], ``counts`` int32 [n],
    ``queries`` f32 [q, dim], all on the GPU."""
    if data.dim() != 2 or data.dtype != torch.float32 or queries.dtype != torch.float32:
        raise ValueError("data and queries must be f32 [n, dim] / [q, dim]")
    if targets.dim() != 2 or targets.dtype != torch.int32 or counts.dtype != torch.int32:
        raise ValueError("targets must be int32 [num_points, row_stride] and counts int32 [num_points]")
    n, dim = data.shape
    q = queries.reshape(-1, dim).contiguous()
    x, t = data.contiguous(), targets.contiguous()
    if t.shape[0] != n or counts.numel() != n:
        raise ValueError(f"neighbour table of {t.shape[0]} rows / {counts.numel()} counts for {n} points")
    ids = torch.empty((q.shape[0], K), dtype=torch.int32, device=x.device)
    d = torch.empty((q.shape[0], K), dtype=torch.float32, device=x.device)
    cmps = torch.empty(q.shape[0], dtype=torch.int32, device=x.device)
    N.check(N.load().tessa_graph_search(_ptr(x), n, dim, _ptr(t), _ptr(counts), t.shape[1], start, _ptr(q), q.shape[0],
                                        L, K, _ptr(ids), _ptr(d), _ptr(cmps), _stream_ptr(stream)), "graph search")
    return ids, d, cmps


def greedy_search_sq8(sq8, targets: torch.Tensor, counts: torch.Tensor, start: int, queries: torch.Tensor, L: int,
                      K: int, stream: torch.cuda.Stream | None = None):
    """``greedy_search`` over SQ8 rows (a tessa.Sq8Matrix on the GPU): row p
    reads as scales[p] * codes[p, :dim] in f32, so the result is the search
    over the dequantized vectors (for sets whose f32 vectors are not kept)."""
    n, dim = sq8.rows, sq8.dim
    q = queries.reshape(-1, dim).contiguous()
    t = targets.contiguous()
    if t.shape[0] != n or counts.numel() != n:
        raise ValueError(f"neighbour table of {t.shape[0]} rows / {counts.numel()} counts for {n} points")
    if q.dtype != torch.float32 or t.dtype != torch.int32 or counts.dtype != torch.int32:
        raise ValueError("queries must be f32, targets and counts int32")
    ids = torch.empty((q.shape[0], K), dtype=torch.int32, device=q.device)
    d = torch.empty((q.shape[0], K), dtype=torch.float32, device=q.device)
    cmps = torch.empty(q.shape[0], dtype=torch.int32, device=q.device)
    N.check(N.load().tessa_graph_search_sq8(_ptr(sq8.codes), _ptr(sq8.scales), sq8.codes.shape[1], n, dim, _ptr(t),
                                            _ptr(counts), t.shape[1], start, _ptr(q), q.shape[0], L, K, _ptr(ids),
                                            _ptr(d), _ptr(cmps), _stream_ptr(stream)), "graph search sq8")
    return ids, d, cmps


def recall_at_k(found: np.ndarray, truth: np.ndarray, k: int) -> float:
    """Mean over queries of (results of the query found among the first k
    ground-truth ids) / k (apps/search_shear_index/src/main.rs:388-411)."""
    f = np.asarray(found)
    g = np.asarray(truth)[:, :k]
    total = 0.0
    for a, b in zip(f, g):
        gt = set(b.tolist())
        total += sum(1 for i in a.tolist() if i in gt) / k
    return total / len(f) if len(f) else 0.0


def robust_prune(data: torch.Tensor, targets: torch.Tensor, counts: torch.Tensor, max_degree: int = 64,
                 max_occlusion: int = 750, alpha: float = 1.2, saturate: bool = False,
                 stream: torch.cuda.Stream | None = None):
    """(targets int32 [n, max_degree] (-1 past the count), counts int32 [n]):
    every row pruned as the reference's final prune does (defaults: the
    reference's max_degree 64, max_occlusion_size 750, alpha 1.2, saturate off)."""
    if data.dim() != 2 or data.dtype != torch.float32:
        raise ValueError("data must be f32 [n, dim]")
    if targets.dim() != 2 or targets.dtype != torch.int32 or counts.dtype != torch.int32:
        raise ValueError("targets must be int32 [num_points, row_stride] and counts int32 [num_points]")
    n, dim = data.shape
    x, t = data.contiguous(), targets.contiguous()
    if t.shape[0] != n or counts.numel() != n:
        raise ValueError(f"neighbour table of {t.shape[0]} rows / {counts.numel()} counts for {n} points")
    out = torch.empty((n, max_degree), dtype=torch.int32, device=x.device)
    cnt = torch.empty(n, dtype=torch.int32, device=x.device)
    N.check(N.load().tessa_robust_prune(_ptr(x), n, dim, _ptr(t), _ptr(counts), t.shape[1], max_degree, max_occlusion,
                                        alpha, 1 if saturate else 0, _ptr(out), _ptr(cnt), _stream_ptr(stream)),
            "robust prune")
    return out, cnt
