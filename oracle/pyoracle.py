"""ctypes wrapper of oracle/libtessa_oracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference semantics used as the parity checker and
as bench.py's cpu_baseline.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module; the product (shear_amd/)
never does.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libtessa_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        P = C.c_void_p
        _lib.orc_sq8_padded_dim.restype = C.c_size_t
        _lib.orc_sq8_padded_dim.argtypes = [C.c_size_t, C.c_size_t]
        _lib.orc_sq8_quantize.restype = C.c_int
        _lib.orc_sq8_quantize.argtypes = [P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_uint, P, P, P, P]
        _lib.orc_sq8_dot_scalar.restype = C.c_int32
        _lib.orc_sq8_dot_scalar.argtypes = [P, P, C.c_size_t]
        _lib.orc_sq8_dot.restype = C.c_int32
        _lib.orc_sq8_dot.argtypes = [P, P, C.c_size_t]
        _lib.orc_sq8_dot_kernel.restype = C.c_int
        _lib.orc_sq8_set_dot_kernel.restype = C.c_int
        _lib.orc_sq8_set_dot_kernel.argtypes = [C.c_int]
        _lib.orc_sq8_leaf_l2.restype = C.c_float
        _lib.orc_sq8_leaf_l2.argtypes = [C.c_int32, C.c_float, C.c_float, C.c_float, C.c_float]
        _lib.orc_sq8_assign_l2.restype = C.c_float
        _lib.orc_sq8_assign_l2.argtypes = [C.c_int32, C.c_float, C.c_float, C.c_float, C.c_float]
        _lib.orc_beats.restype = C.c_int
        _lib.orc_beats.argtypes = [C.c_float, C.c_uint32, C.c_float, C.c_uint32]
        _lib.orc_rowtopk_push.restype = None
        _lib.orc_rowtopk_push.argtypes = [C.c_uint32, C.c_float, C.c_uint32, P, P, P]
        _lib.orc_leaf_topk_batch.restype = C.c_int
        _lib.orc_leaf_topk_batch.argtypes = [P, P, P, P, C.c_size_t, C.c_size_t, P, P, P, P, C.c_size_t,
                                             C.c_uint32, P, P, C.c_int]
        _lib.orc_hash64.restype = C.c_uint64
        _lib.orc_hash64.argtypes = [C.c_uint64]
        _lib.orc_assign_tie_key.restype = C.c_uint64
        _lib.orc_assign_tie_key.argtypes = [C.c_uint32, C.c_uint32]
        for name in ("orc_assign_replay", "orc_assign_strict"):
            fn = getattr(_lib, name)
            fn.restype = C.c_int
            fn.argtypes = [P, P, P, P, C.c_size_t, C.c_size_t, P, P, P, P, P, P, P, P, C.c_size_t, P, P, C.c_int]
        _lib.orc_assign_before.restype = C.c_int
        _lib.orc_assign_before.argtypes = [C.c_float, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32]
        _lib.orc_adaptive_psamp.restype = C.c_float
        _lib.orc_adaptive_psamp.argtypes = [C.c_float, C.c_uint32, C.c_uint32]
        _lib.orc_meaningful_split.restype = C.c_int
        _lib.orc_meaningful_split.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
        _lib.orc_sort_unique.restype = None
        _lib.orc_sort_unique.argtypes = [P, P]
        _lib.orc_sample_retry_leaders.restype = None
        _lib.orc_sample_retry_leaders.argtypes = [P, C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint32, P]
        _lib.orc_hash_rank_leaders.restype = None
        _lib.orc_hash_rank_leaders.argtypes = [P, C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint32, C.c_uint32, P]
        _lib.orc_subtree_root_seed.restype = C.c_uint64
        _lib.orc_subtree_root_seed.argtypes = [C.c_uint64] * 5
        _lib.orc_subtree_partition.restype = C.c_int
        _lib.orc_subtree_partition.argtypes = [P, P, P, C.c_size_t, C.c_size_t, C.POINTER(SubtreeCfg), P, P, P,
                                               P, P, P]
        _lib.orc_compute_hash.restype = C.c_uint16
        _lib.orc_compute_hash.argtypes = [P, P, C.c_uint]
        _lib.orc_flush_compact_topk_into_edges.restype = C.c_longlong
        _lib.orc_flush_compact_topk_into_edges.argtypes = [P, C.c_size_t, C.c_size_t, P, P, P, C.c_size_t,
                                                           C.c_size_t, C.c_uint, P, C.c_size_t, P]
        _lib.orc_hashprune_reduce.restype = C.c_int
        _lib.orc_hashprune_reduce.argtypes = [C.c_size_t, C.c_size_t, P, C.c_size_t, P, P, P, P, P]
        _lib.orc_hashprune_rhalf_reduce.restype = C.c_int
        _lib.orc_hashprune_rhalf_reduce.argtypes = [C.c_size_t, C.c_size_t, P, C.c_size_t, C.c_int, C.c_uint,
                                                    C.c_uint, C.c_float, P, P, P, P, P, P]
        _lib.orc_d0_assign.restype = C.c_int
        _lib.orc_d0_assign.argtypes = [P, P, P, P, C.c_size_t, C.c_size_t, P, P, P, P, C.c_size_t, C.c_size_t, P, P,
                                       P, P]
        _lib.orc_robust_prune.restype = C.c_int
        _lib.orc_robust_prune.argtypes = [P, C.c_size_t, C.c_size_t, P, P, C.c_size_t, C.c_size_t, C.c_size_t,
                                          C.c_float, C.c_int, P, P]
        _lib.orc_greedy_search.restype = C.c_int
        _lib.orc_greedy_search.argtypes = [P, C.c_size_t, C.c_size_t, P, P, C.c_size_t, C.c_uint32, P, C.c_size_t,
                                           C.c_size_t, C.c_size_t, P, P, P]
    return _lib


class SubtreeCfg(C.Structure):
    """orc_subtree_cfg (tessa_oracle.h)."""

    _fields_ = [
        ("root_leaders", C.c_void_p),
        ("root_leader_count", C.c_uint32),
        ("root_depth", C.c_uint32),
        ("max_depth", C.c_uint32),
        ("max_leaders", C.c_uint32),
        ("fanout_second", C.c_uint32),
        ("leaf_min", C.c_uint32),
        ("leaf_max", C.c_uint32),
        ("small_node_limit", C.c_uint32),
        ("large_scratch_rows", C.c_uint64),
        ("max_leaf_count", C.c_uint64),
        ("max_leaf_rows", C.c_uint64),
        ("psamp_fraction", C.c_float),
        ("seed", C.c_uint64),
        ("trace_min_members", C.c_uint32),
        ("trace", C.c_void_p),
    ]


class PassTrace(C.Structure):
    """orc_pass_trace (tessa_oracle.h)."""

    _fields_ = [
        ("passes", C.POINTER(C.c_uint32)),
        ("pass_len", C.c_size_t),
        ("pass_cap", C.c_size_t),
        ("rows", C.POINTER(C.c_uint32)),
        ("row_len", C.c_size_t),
        ("row_cap", C.c_size_t),
    ]


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def padded_dim(dim: int, k_align: int = 16) -> int:
    return int(lib().orc_sq8_padded_dim(dim, k_align))


def quantize(x: np.ndarray, k_align: int = 16, bits: int = 8):
    """-> (codes int8 [rows, pd], scales f32, norms f32); ValueError on non-finite."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, dim = x.shape
    pd = padded_dim(dim, k_align)
    codes = np.zeros((rows, pd), dtype=np.int8)
    scales = np.zeros(rows, dtype=np.float32)
    norms = np.zeros(rows, dtype=np.float32)
    bad = C.c_size_t(0)
    rc = lib().orc_sq8_quantize(_p(x), rows, dim, pd, bits, _p(codes), _p(scales), _p(norms), C.byref(bad))
    if rc == -1:
        raise ValueError(f"SQ-int8 cannot quantize non-finite value (row {bad.value})")
    if rc != 0:
        raise ValueError(f"invalid quantize arguments (rc={rc})")
    return codes, scales, norms


def dot(a: np.ndarray, b: np.ndarray, scalar: bool = False) -> int:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    fn = lib().orc_sq8_dot_scalar if scalar else lib().orc_sq8_dot
    return int(fn(_p(a), _p(b), a.size))


def set_dot_kernel(k: int) -> int:
    return int(lib().orc_sq8_set_dot_kernel(k))


def dot_kernel() -> int:
    return int(lib().orc_sq8_dot_kernel())


def leaf_l2(dot_: int, rs: float, rn: float, cs: float, cn: float) -> np.float32:
    return np.float32(lib().orc_sq8_leaf_l2(dot_, rs, rn, cs, cn))


def assign_l2(dot_: int, ps: float, pn: float, ls: float, ln: float) -> np.float32:
    return np.float32(lib().orc_sq8_assign_l2(dot_, ps, pn, ls, ln))


def beats(dc: float, idc: int, ds: float, ids: int) -> bool:
    return bool(lib().orc_beats(dc, idc, ds, ids))


class RowTopK:
    """leaf_build.rs:887-957 via the oracle's push."""

    def __init__(self):
        self.d = np.full(32, np.inf, dtype=np.float32)
        self.ids = np.full(32, 0xFFFFFFFF, dtype=np.uint32)
        self.len = C.c_uint32(0)

    def push(self, k: int, dist: float, target: int):
        lib().orc_rowtopk_push(k, dist, target, _p(self.d), _p(self.ids), C.byref(self.len))

    def items(self):
        n = self.len.value
        return list(zip(self.ids[:n].tolist(), self.d[:n].tolist()))


def leaf_topk(codes, scales, norms, global_ids, members, member_offsets, member_counts, k, threads=0):
    """Leaf operator over replay layouts; returns (ids u32, dists f32) flat."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    norms = np.ascontiguousarray(norms, dtype=np.float32)
    gids = np.ascontiguousarray(global_ids, dtype=np.uint32)
    members = np.ascontiguousarray(members, dtype=np.uint32)
    moff = np.ascontiguousarray(member_offsets, dtype=np.uint64)
    mcnt = np.ascontiguousarray(member_counts, dtype=np.uint32)
    ooff = np.zeros(len(mcnt), dtype=np.uint64)
    if len(mcnt) > 1:
        ooff[1:] = np.cumsum(mcnt[:-1].astype(np.uint64) * np.uint64(k))
    total = int(mcnt.astype(np.int64).sum()) * k
    out_ids = np.zeros(total, dtype=np.uint32)
    out_d = np.zeros(total, dtype=np.float32)
    rc = lib().orc_leaf_topk_batch(_p(codes), _p(scales), _p(norms), _p(gids), codes.shape[0], codes.shape[1],
                                   _p(members), _p(moff), _p(mcnt), _p(ooff), len(mcnt), k, _p(out_ids),
                                   _p(out_d), threads)
    if rc != 0:
        raise ValueError(f"oracle leaf_topk failed rc={rc}")
    return out_ids, out_d


def _assign(fn_name, codes, scales, norms, global_ids, members, leaders, member_offsets, member_counts,
            leader_offsets, leader_counts, r_h, threads=0):
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    a32 = lambda x: np.ascontiguousarray(x, dtype=np.uint32)  # noqa: E731
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    norms = np.ascontiguousarray(norms, dtype=np.float32)
    gids, mem, lead = a32(global_ids), a32(members), a32(leaders)
    mo, mc, lo, lc, rh = a32(member_offsets), a32(member_counts), a32(leader_offsets), a32(leader_counts), a32(r_h)
    oo = np.zeros(len(mc), dtype=np.uint64)
    if len(mc) > 1:
        oo[1:] = np.cumsum(mc[:-1].astype(np.uint64) * rh[:-1].astype(np.uint64))
    total = int((mc.astype(np.int64) * rh.astype(np.int64)).sum())
    out_ids = np.zeros(total, dtype=np.uint32)
    out_d = np.zeros(total, dtype=np.float32)
    rc = getattr(lib(), fn_name)(_p(codes), _p(scales), _p(norms), _p(gids), codes.shape[0], codes.shape[1],
                                 _p(mem), _p(lead), _p(mo), _p(mc), _p(lo), _p(lc), _p(rh), _p(oo), len(mc),
                                 _p(out_ids), _p(out_d), threads)
    if rc != 0:
        raise ValueError(f"oracle {fn_name} failed rc={rc}")
    return out_ids, out_d


def assign_replay(*args, **kw):
    return _assign("orc_assign_replay", *args, **kw)


def assign_strict(*args, **kw):
    return _assign("orc_assign_strict", *args, **kw)


def hash64(x: int) -> int:
    return int(lib().orc_hash64(x))


def assign_tie_key(point: int, leader: int) -> int:
    return int(lib().orc_assign_tie_key(point, leader))


def assign_before(d: float, point: int, leader: int, od: float, oleader: int) -> bool:
    return bool(lib().orc_assign_before(d, point, leader, od, oleader))


def adaptive_psamp(base: float, n: int, depth: int) -> np.float32:
    return np.float32(lib().orc_adaptive_psamp(base, n, depth))


def meaningful_split(parent: int, max_child: int, terminal: int) -> bool:
    return bool(lib().orc_meaningful_split(parent, max_child, terminal))


def sort_unique(v) -> np.ndarray:
    a = np.ascontiguousarray(v, np.uint32).copy()
    n = C.c_uint32(len(a))
    lib().orc_sort_unique(_p(a), C.byref(n))
    return a[: n.value]


def sample_retry_leaders(rows, num_leaders: int, seed: int, attempt: int) -> np.ndarray:
    rows = np.ascontiguousarray(rows, np.uint32)
    out = np.zeros(num_leaders, np.uint32)
    lib().orc_sample_retry_leaders(_p(rows), len(rows), num_leaders, seed, attempt, _p(out))
    return out


def hash_rank_leaders(pts, num_leaders: int, seed: int, attempt: int, depth: int) -> np.ndarray:
    pts = np.ascontiguousarray(pts, np.uint32)
    out = np.zeros(num_leaders, np.uint32)
    lib().orc_hash_rank_leaders(_p(pts), len(pts), num_leaders, seed, attempt, depth, _p(out))
    return out


def subtree_root_seed(random_seed: int, depth: int, point_count: int, parent_points: int,
                      min_recurse_size: int) -> int:
    return int(lib().orc_subtree_root_seed(random_seed, depth, point_count, parent_points, min_recurse_size))


COUNTER_WORDS = 159


def subtree_partition(codes, scales, norms, *, seed: int, root_depth: int = 0, max_depth: int = 10,
                      max_leaders: int = 128, fanout_second: int = 1, leaf_min: int = 64, leaf_max: int = 256,
                      small_node_limit: int = 4096, psamp_fraction: float = 0.001, root_leaders=None,
                      large_scratch_rows: int | None = None, max_leaf_count: int | None = None,
                      max_leaf_rows: int | None = None, trace_min_members: int = 0):
    """-> (leaves: list of u32 arrays (resident rows, in order), counters u64[159]).

    With trace_min_members > 0 a third value is returned: the COUNT passes of
    nodes with at least that many rows, as a list of dicts (depth, attempt,
    fanout, members, leaders; resident rows), in the oracle's walk order."""
    codes = np.ascontiguousarray(codes, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    norms = np.ascontiguousarray(norms, np.float32)
    rows, pd = codes.shape
    famp = max(1, min(fanout_second, 4))
    roots = np.zeros(0, np.uint32) if root_leaders is None else np.ascontiguousarray(root_leaders, np.uint32)
    mlr = max_leaf_rows if max_leaf_rows is not None else max(rows * famp, 1)
    mlc = max_leaf_count if max_leaf_count is not None else max(rows * famp, 1)
    trace = PassTrace()
    cfg = SubtreeCfg(roots.ctypes.data if len(roots) else None, len(roots), root_depth, max_depth, max_leaders,
                     fanout_second, leaf_min, leaf_max, small_node_limit,
                     large_scratch_rows if large_scratch_rows is not None else max(rows, 1) * famp,
                     mlc, mlr, np.float32(psamp_fraction).item(), seed & (2**64 - 1), trace_min_members,
                     C.cast(C.pointer(trace), C.c_void_p) if trace_min_members > 0 else None)
    leaf_rows = np.zeros(max(mlr, 1), np.uint32)
    starts = np.zeros(max(mlc, 1), np.uint64)
    sizes = np.zeros(max(mlc, 1), np.uint64)
    ctr = np.zeros(COUNTER_WORDS, np.uint64)
    lc = C.c_uint64(0)
    lr = C.c_uint64(0)
    rc = lib().orc_subtree_partition(_p(codes), _p(scales), _p(norms), rows, pd, C.byref(cfg), _p(leaf_rows),
                                     _p(starts), _p(sizes), _p(ctr), C.byref(lc), C.byref(lr))
    passes = None
    if trace_min_members > 0:
        passes = []
        w = np.ctypeslib.as_array(trace.passes, (trace.pass_len,)).copy() if trace.pass_len else np.zeros(0, np.uint32)
        r = np.ctypeslib.as_array(trace.rows, (trace.row_len,)).copy() if trace.row_len else np.zeros(0, np.uint32)
        lib().orc_pass_trace_free(C.byref(trace))
        off = 0
        for i in range(0, len(w), 5):
            depth, attempt, fanout, nm, nl = (int(v) for v in w[i:i + 5])
            passes.append(dict(depth=depth, attempt=attempt, fanout=fanout, members=r[off:off + nm],
                               leaders=r[off + nm:off + nm + nl]))
            off += nm + nl
    if rc != 0:
        raise ValueError(f"orc_subtree_partition failed: {rc}")
    n_leaves = min(lc.value, mlc)
    if ctr[7] != 0:
        return (None, ctr, passes) if trace_min_members > 0 else (None, ctr)
    leaves = [leaf_rows[int(starts[i]): int(starts[i]) + int(sizes[i])].copy() for i in range(n_leaves)]
    return (leaves, ctr, passes) if trace_min_members > 0 else (leaves, ctr)


# spill_hashprune.rs:137-145 SpillRecord16 (little-endian, 16 bytes)
EDGE_DTYPE = np.dtype([("src", "<u4"), ("dst", "<u4"), ("hash", "<u2"), ("flags", "<u2"), ("dist", "<f4")])


def compute_hash(sketch_p, sketch_c, m_bits: int) -> int:
    sp = np.ascontiguousarray(sketch_p, np.float32)
    sc = np.ascontiguousarray(sketch_c, np.float32)
    return int(lib().orc_compute_hash(_p(sp), _p(sc), m_bits))


class EdgeError(ValueError):
    def __init__(self, code: int, point: int):
        super().__init__(f"orc_flush_compact_topk_into_edges: {code} (point {point})")
        self.code = code
        self.point = point


def flush_compact_topk_into_edges(point_ids, k: int, topk_ids, topk_dists, sketches, m_bits: int):
    """One CompactTopKBatch -> SpillRecord16 records (EDGE_DTYPE array).
    sketches: [sketch_rows, width] f32, row = global point id."""
    pids = np.ascontiguousarray(point_ids, np.uint32)
    ids = np.ascontiguousarray(topk_ids, np.uint32)
    d = np.ascontiguousarray(topk_dists, np.float32)
    sk = np.ascontiguousarray(sketches, np.float32)
    rows = len(pids)
    out = np.zeros(max(2 * rows * k, 1), EDGE_DTYPE)
    bad = C.c_uint32(0)
    n = lib().orc_flush_compact_topk_into_edges(_p(pids), rows, k, _p(ids), _p(d), _p(sk), sk.shape[0],
                                                sk.shape[1], m_bits, _p(out), len(out), C.byref(bad))
    if n < 0:
        raise EdgeError(int(n), bad.value)
    return out[:n]


def hashprune_reduce(num_points: int, l_max: int, records: np.ndarray):
    """HashPrune reservoirs after inserting `records` (EDGE_DTYPE) in order:
    (targets [num_points, l_max] u32, hashes u16, dists f32, counts [num_points] u32),
    each row's slots in ascending hash order, unused slots 0xFFFFFFFF / 0 / 0."""
    rec = np.ascontiguousarray(records, EDGE_DTYPE)
    t = np.zeros((num_points, l_max), np.uint32)
    hs = np.zeros((num_points, l_max), np.uint16)
    d = np.zeros((num_points, l_max), np.float32)
    cnt = np.zeros(num_points, np.uint32)
    bad = C.c_uint32(0)
    rc = lib().orc_hashprune_reduce(num_points, l_max, _p(rec), len(rec), _p(t), _p(hs), _p(d), _p(cnt),
                                    C.byref(bad))
    if rc != 0:
        raise ValueError(f"orc_hashprune_reduce: {rc} (record {bad.value})")
    return t, hs, d, cnt


RHALF_MODES = {"rhalf-hash-slot-1": 1, "rhalf-distance-first-q3": 2, "rhalf-soft-tier-q3": 3,
               "rhalf-hard-tier-q3": 4}


def hashprune_rhalf_reduce(num_points: int, l_max: int, records: np.ndarray, mode: str = "rhalf-soft-tier-q3",
                           hash_quota: int = 0, row_cap: int = 0, priority_alpha: float = 0.0):
    """HashPrune with a named R-half backfill policy (hash_prune_backfill.rs,
    hash_prune.rs:2601-2682): (targets [num_points, l_max] u32, hashes u16,
    dists f32, counts [num_points] u32 (primaries + shortlist), primary counts);
    each row's primaries in ascending hash order, then its shortlist in
    priority order.  row_cap 0 = none; priority_alpha 0 = 1.1."""
    rec = np.ascontiguousarray(records, EDGE_DTYPE)
    t = np.zeros((num_points, l_max), np.uint32)
    hs = np.zeros((num_points, l_max), np.uint16)
    d = np.zeros((num_points, l_max), np.float32)
    cnt = np.zeros(num_points, np.uint32)
    pcnt = np.zeros(num_points, np.uint32)
    bad = C.c_uint32(0)
    rc = lib().orc_hashprune_rhalf_reduce(num_points, l_max, _p(rec), len(rec), RHALF_MODES[mode], hash_quota,
                                          row_cap, priority_alpha, _p(t), _p(hs), _p(d), _p(cnt), _p(pcnt),
                                          C.byref(bad))
    if rc != 0:
        raise ValueError(f"orc_hashprune_rhalf_reduce: {rc} (record {bad.value})")
    return t, hs, d, cnt, pcnt


def graph_bytes(start: int, num_frozen: int, rows) -> bytes:
    """DirectMemGraphWriter file bytes (index/inmem_index/pipnn_oom_writer.rs:35-72):
    header (index_size u64, max_degree u32, start u32, num_frozen_pts u64), then
    per row its degree (u32) and ids (u32), little-endian."""
    body = b"".join(np.uint32(len(r)).tobytes() + np.asarray(r, "<u4").tobytes() for r in rows)
    max_degree = max((len(r) for r in rows), default=0)
    head = np.array([(24 + len(body), max_degree, start, num_frozen)], dtype=np.dtype("<u8,<u4,<u4,<u8")).tobytes()
    return head + body


def greedy_search(data: np.ndarray, targets: np.ndarray, counts: np.ndarray, start: int, queries: np.ndarray,
                  L: int, K: int):
    """Greedy search over the neighbour table (targets u32 [n, row_stride],
    counts [n]) from `start` with search list L (algorithm/search/search.rs:137-233):
    (ids u32 [q, K], squared-L2 f32 [q, K], distance evaluations u32 [q])."""
    x = np.ascontiguousarray(data, np.float32)
    t = np.ascontiguousarray(targets).view(np.uint32) if np.asarray(targets).dtype.itemsize == 4 else None
    if t is None or t.ndim != 2:
        raise ValueError("targets must be a 4-byte [n, row_stride] array")
    c = np.ascontiguousarray(counts).astype(np.uint32)
    q = np.ascontiguousarray(queries, np.float32).reshape(-1, x.shape[1])
    ids = np.zeros((len(q), K), np.uint32)
    d = np.zeros((len(q), K), np.float32)
    cmps = np.zeros(len(q), np.uint32)
    rc = lib().orc_greedy_search(_p(x), x.shape[0], x.shape[1], _p(t), _p(c), t.shape[1], start, _p(q), len(q), L, K,
                                 _p(ids), _p(d), _p(cmps))
    if rc != 0:
        raise ValueError(f"orc_greedy_search: {rc}")
    return ids, d, cmps


def d0_assign(codes, scales, norms, global_ids, leader_codes, leader_scales, leader_norms, leader_ids, fanout):
    """Global D0 assignment (compute_backend.rs:18016-18511): (child u32 [rows, fanout]
    leader indices, child_offsets u64 [leaders + 1], child_points u32 grouped by
    child, rows ascending)."""
    c = np.ascontiguousarray(codes, np.int8)
    lc = np.ascontiguousarray(leader_codes, np.int8)
    rows, pd = c.shape
    nl = lc.shape[0]
    s, n = np.ascontiguousarray(scales, np.float32), np.ascontiguousarray(norms, np.float32)
    ls, ln = np.ascontiguousarray(leader_scales, np.float32), np.ascontiguousarray(leader_norms, np.float32)
    g = np.ascontiguousarray(global_ids, np.uint32)
    lid = np.ascontiguousarray(leader_ids, np.uint32)
    child = np.zeros((rows, fanout), np.uint32)
    point = np.zeros((rows, fanout), np.uint32)
    offs = np.zeros(nl + 1, np.uint64)
    pts = np.zeros(rows * fanout, np.uint32)
    rc = lib().orc_d0_assign(_p(c), _p(s), _p(n), _p(g), rows, pd, _p(lc), _p(ls), _p(ln), _p(lid), nl, fanout,
                             _p(child), _p(point), _p(offs), _p(pts))
    if rc != 0:
        raise ValueError(f"orc_d0_assign: {rc}")
    return child, offs, pts


def robust_prune(data: np.ndarray, targets: np.ndarray, counts: np.ndarray, max_degree: int = 64,
                 max_occlusion: int = 750, alpha: float = 1.2, saturate: bool = False):
    """Final RobustPrune of every row (pipnn_builder.rs:287-330, prune.rs:17-214):
    (targets u32 [n, max_degree], counts u32 [n])."""
    x = np.ascontiguousarray(data, np.float32)
    t = np.ascontiguousarray(targets).view(np.uint32)
    c = np.ascontiguousarray(counts).astype(np.uint32)
    out = np.zeros((x.shape[0], max_degree), np.uint32)
    cnt = np.zeros(x.shape[0], np.uint32)
    rc = lib().orc_robust_prune(_p(x), x.shape[0], x.shape[1], _p(t), _p(c), t.shape[1], max_degree, max_occlusion,
                                alpha, 1 if saturate else 0, _p(out), _p(cnt))
    if rc != 0:
        raise ValueError(f"orc_robust_prune: {rc}")
    return out, cnt
