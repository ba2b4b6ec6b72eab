"""ctypes binding of libtessa_hip.so (the C ABI in include/tessa_hip.h).

The library is the product path: when it is missing or fails to load, every
entry point raises -- there is no CPU fallback anywhere in this package.
Device buffers are passed as raw device pointers (torch tensors on `cuda` are
used only as allocations and streams).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtessa_hip.so"

# enum tessa_counter / overflow bits (include/tessa_hip.h)
COUNTER_WORDS = 32
C_OVERFLOW_FLAGS = 0
C_LEAF_ROWS = 1
C_LEAF_MFMA_TILES = 2
C_LEAF_EXACT_ROWS = 3
C_LEAF_FALLBACK_ROWS = 4
C_LEAF_LIST_OVERFLOW_ROWS = 5
C_LEAF_GAP_FALLBACK_ROWS = 6
C_LEAF_REFINES = 7
C_LEAF_SURVIVORS = 8
C_LEAF_FINAL_CANDIDATES = 9
C_ASSIGN_ROWS = 10
C_ASSIGN_PAIRS = 11
C_ASSIGN_TIE_EVENTS = 12
C_LEAF_CHAIN_ROWS = 13

EXEC_EXACT = 1
EXEC_MFMA = 2

TESSA_OK = 0


class TessaStatus(C.Structure):
    _fields_ = [
        ("code", C.c_int32),
        ("reserved", C.c_uint32),
        ("overflow_flags", C.c_uint64),
        ("msg", C.c_char * 512),
    ]


class TessaCaps(C.Structure):
    _fields_ = [
        ("device", C.c_int32),
        ("compute_units", C.c_int32),
        ("max_threads_per_block", C.c_int32),
        ("lds_bytes_per_block", C.c_int32),
        ("hbm_bytes", C.c_uint64),
        ("arch", C.c_char * 64),
        ("supported", C.c_int32),
        ("max_leaf_rows", C.c_int32),
        ("max_k", C.c_int32),
        ("max_padded_dim", C.c_int32),
    ]


class Sq8View(C.Structure):
    _fields_ = [
        ("codes", C.c_void_p),
        ("scales", C.c_void_p),
        ("norms", C.c_void_p),
        ("global_ids", C.c_void_p),
        ("rows", C.c_uint64),
        ("dim", C.c_uint32),
        ("padded_dim", C.c_uint32),
    ]


class LeafBatch(C.Structure):
    _fields_ = [
        ("members", C.c_void_p),
        ("member_offsets", C.c_void_p),
        ("member_counts", C.c_void_p),
        ("output_offsets", C.c_void_p),
        ("leaf_count", C.c_uint32),
        ("max_leaf_rows", C.c_uint32),
        ("k", C.c_uint32),
        ("executor", C.c_uint32),
        ("debug_rerun_every", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class AssignBatch(C.Structure):
    _fields_ = [
        ("members", C.c_void_p),
        ("leaders", C.c_void_p),
        ("member_offsets", C.c_void_p),
        ("member_counts", C.c_void_p),
        ("leader_offsets", C.c_void_p),
        ("leader_counts", C.c_void_p),
        ("r_h", C.c_void_p),
        ("output_offsets", C.c_void_p),
        ("task_count", C.c_uint32),
        ("max_members", C.c_uint32),
    ]


class TessaConfig(C.Structure):
    _fields_ = [("device", C.c_int32), ("reserved", C.c_uint32)]


class HashPruneBackfill(C.Structure):
    _fields_ = [("mode", C.c_uint32), ("hash_quota", C.c_uint32), ("max_backfill_per_row", C.c_uint32),
                ("soft_tier_priority_alpha", C.c_float)]


# Subtree counters at the reference's indices (enum tessa_subtree_counter).
SUBTREE_COUNTER_WORDS = 159
P_OVERFLOW_FLAGS = 7
P_PARTITION_POPS = 8
P_OUTPUT_ROWS = 12
P_OUTPUT_LEAF_COUNT = 13
P_ASSIGNMENT_PASSES = 14
P_MAX_ACTIVE = 15
P_EFFECTIVE_ROOT_FANOUT = 17
P_EFFECTIVE_DEEPER_FANOUT = 18
P_FANOUT_ASSIGNMENT_SLOTS = 19
P_REPLICATED_ROWS = 20
P_UNIQUE_RESIDENT_ROWS = 21
P_LARGE_NODE_CLAIMS = 27
P_LARGE_NODE_SPLITS = 28
P_LARGE_NODE_ROWS = 29
P_LARGE_NODE_MAX_ROWS = 30
P_LEAF_SIZE_MIN = 33
P_LEAF_SIZE_MAX = 34
P_LEAF_SIZE_SUM = 35
P_LEAF_SIZE_COUNT = 36
P_PARTITION_LEVEL_ROUNDS = 119
# phase clocks of the persistent partition walk (ticks of the 100 MHz wall clock)
P_PARTITION_BUSY_CLOCKS = 120
P_PARTITION_WAIT_CLOCKS = 121
P_LARGE_COUNT_DISTANCE_CLOCKS = 140
P_LARGE_COUNT_COMMIT_CLOCKS = 141
P_LARGE_SCATTER_CLOCKS = 142
P_LARGE_PUBLISH_CLOCKS = 143
P_CLOCK_WORDS = (120, 121, 140, 141, 142, 143)
P_LARGE_SPLIT_RETRIES = 130
P_LARGE_BALANCED_FALLBACKS = 131
P_LARGE_PHYSICAL_TILES = 145
P_LEAF_SQ8_WMMA_TILES = 158

PLAN_FALLBACK_UNSUPPORTED_K = 1 << 2
PLAN_FALLBACK_UNSUPPORTED_FANOUT = 1 << 3
PLAN_FALLBACK_UNSUPPORTED_LEADERS = 1 << 4
PLAN_FALLBACK_WORKSPACE = 1 << 5


class SubtreePlan(C.Structure):
    _fields_ = [
        ("supported", C.c_int32),
        ("fallback_reason_flags", C.c_uint32),
        ("overflow_flags", C.c_uint64),
        ("leaf_min", C.c_uint32),
        ("leaf_target", C.c_uint32),
        ("leaf_max", C.c_uint32),
        ("small_node_limit", C.c_uint32),
        ("effective_root_fanout", C.c_uint32),
        ("effective_deeper_fanout", C.c_uint32),
        ("fanout_amplification", C.c_uint32),
        ("large_child_slots", C.c_uint32),
        ("max_queue_nodes", C.c_uint64),
        ("max_leaf_count", C.c_uint64),
        ("max_leaf_rows", C.c_uint64),
        ("large_scratch_rows", C.c_uint64),
        ("required_bytes", C.c_uint64),
        ("budget_bytes", C.c_uint64),
    ]


class SubtreeRequest(C.Structure):
    _fields_ = [
        ("root_leaders", C.c_void_p),
        ("root_leader_count", C.c_uint32),
        ("root_depth", C.c_uint32),
        ("seed", C.c_uint64),
        ("leaf_knn", C.c_uint32),
        ("fanout_second", C.c_uint32),
        ("max_depth", C.c_uint32),
        ("max_leaders", C.c_uint32),
        ("leaf_min", C.c_uint32),
        ("leaf_max", C.c_uint32),
        ("small_node_limit", C.c_uint32),
        ("psamp_fraction", C.c_float),
        ("executor", C.c_uint32),
        ("partition_only", C.c_uint32),
        ("max_leaf_count", C.c_uint64),
        ("max_leaf_rows", C.c_uint64),
    ]


class SubtreeOutput(C.Structure):
    _fields_ = [
        ("leaf_row_ids", C.c_void_p),
        ("leaf_starts", C.c_void_p),
        ("leaf_sizes", C.c_void_p),
        ("topk_ids", C.c_void_p),
        ("topk_dists", C.c_void_p),
        ("counters", C.c_void_p),
        ("leaf_counters", C.c_void_p),
        ("leaf_count", C.c_uint64),
        ("leaf_rows", C.c_uint64),
        ("k", C.c_uint32),
        ("levels", C.c_uint32),
        ("partition_ms", C.c_float),
        ("leaf_ms", C.c_float),
    ]


class RootsRequest(C.Structure):
    _fields_ = [("rows", C.c_void_p), ("root_offsets", C.c_void_p), ("root_seeds", C.c_void_p),
                ("root_count", C.c_uint32), ("root_depth", C.c_uint32), ("fanout_second", C.c_uint32),
                ("max_depth", C.c_uint32), ("max_leaders", C.c_uint32), ("leaf_min", C.c_uint32),
                ("leaf_max", C.c_uint32), ("small_node_limit", C.c_uint32), ("psamp_fraction", C.c_float),
                ("reserved", C.c_uint32), ("max_leaf_count", C.c_uint64), ("max_leaf_rows", C.c_uint64)]


class RootsOutput(C.Structure):
    _fields_ = [("leaf_rows", C.c_void_p), ("leaf_starts", C.c_void_p), ("leaf_sizes", C.c_void_p),
                ("leaf_roots", C.c_void_p), ("leaf_depths", C.c_void_p), ("counters", C.c_void_p), ("leaf_count", C.c_uint64), ("leaf_rows_total", C.c_uint64),
                ("levels", C.c_uint32), ("partition_ms", C.c_float)]


class SubtreeHostResult(C.Structure):
    _fields_ = [
        ("leaf_row_ids", C.c_void_p),
        ("leaf_starts", C.c_void_p),
        ("leaf_sizes", C.c_void_p),
        ("topk_ids", C.c_void_p),
        ("topk_dists", C.c_void_p),
        ("counters", C.c_void_p),
        ("leaf_counters", C.c_void_p),
        ("leaf_count", C.c_uint64),
        ("leaf_rows", C.c_uint64),
        ("k", C.c_uint32),
        ("levels", C.c_uint32),
        ("partition_ms", C.c_float),
        ("leaf_ms", C.c_float),
    ]


class EdgeRecord(C.Structure):
    """tessa_edge_record: SpillRecord16 (spill_hashprune.rs:137-145)."""

    _fields_ = [
        ("src", C.c_uint32),
        ("dst", C.c_uint32),
        ("hash", C.c_uint16),
        ("flags", C.c_uint16),
        ("dist", C.c_float),
    ]


class SketchView(C.Structure):
    _fields_ = [
        ("rows", C.c_void_p),
        ("sketch_rows", C.c_uint64),
        ("width", C.c_uint32),
        ("m_bits", C.c_uint32),
    ]


class ResidentAdmission(C.Structure):
    _fields_ = [("plan", SubtreePlan), ("resident_device_bytes", C.c_uint64),
                ("device_admission_required_bytes", C.c_uint64), ("device_admission_budget_bytes", C.c_uint64)]


class D0Thresholds(C.Structure):
    _fields_ = [("c_gpu", C.c_uint64), ("c_high", C.c_uint64), ("c_target", C.c_uint64), ("c_low", C.c_uint64)]


class D0LeaderPlan(C.Structure):
    _fields_ = [("k_capacity", C.c_uint64), ("k_initial", C.c_uint64), ("root_leader_cap", C.c_uint64),
                ("source", C.c_uint32)]


class D0ChildSummary(C.Structure):
    _fields_ = [(f, C.c_uint64) for f in ("max_rows", "p50_rows", "p95_rows", "p99_rows", "oversized_count",
                                          "small_count", "small_rows")]


RESIDENT_F32, RESIDENT_SQ8, RESIDENT_SQ4 = 0, 1, 2
D0_LEADER_SOURCES = ("capacity", "quality_floor", "root_leader_cap")


class CapturedAssignment(C.Structure):
    _fields_ = [("depth", C.c_uint32), ("retry", C.c_uint32), ("r_h", C.c_uint32), ("padded_dim", C.c_uint32),
                ("member_count", C.c_uint32), ("leader_count", C.c_uint32), ("member_offset", C.c_uint64),
                ("leader_offset", C.c_uint64)]


class TierLiftConfig(C.Structure):
    _fields_ = [("num_points", C.c_uint64), ("shard_points", C.c_uint64), ("host_budget_bytes", C.c_uint64),
                ("staging_records", C.c_uint64), ("spill_base", C.c_char_p), ("l_max", C.c_uint32),
                ("threads", C.c_uint32), ("expected_records", C.c_uint64)]


class TierLiftStats(C.Structure):
    _fields_ = [(f, C.c_uint64) for f in ("records", "pushes", "host_peak_bytes", "spilled_records",
                                          "spilled_bytes", "segments", "reread_records")] + [
        ("shards", C.c_uint32), ("threads", C.c_uint32), ("route_s", C.c_double), ("spill_s", C.c_double),
        ("reduce_s", C.c_double), ("unique_records", C.c_uint64)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


# Every symbol include/tessa_hip.h declares, with its ctypes signature.
_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
SIGNATURES = {
    "tessa_abi_version": (_U32, []),
    "tessa_probe_mfma_rate": (TessaStatus, [_U32, _U32, _U64, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "tessa_overflow_labels": (None, [_U64, C.c_char_p, C.c_size_t]),
    "tessa_query_caps": (TessaStatus, [C.c_int32, C.POINTER(TessaCaps)]),
    "tessa_leaf_topk": (TessaStatus, [C.POINTER(Sq8View), C.POINTER(LeafBatch), _P, _P, _P, _P]),
    "tessa_leaf_topk_noalloc": (TessaStatus, [C.POINTER(Sq8View), C.POINTER(LeafBatch), _P, _P, _P, _P]),
    "tessa_leaf_topk_profiled": (
        TessaStatus,
        [C.POINTER(Sq8View), C.POINTER(LeafBatch), _P, _P, _P, _P, C.POINTER(C.c_float)],
    ),
    "tessa_assign_replay": (TessaStatus, [C.POINTER(Sq8View), C.POINTER(AssignBatch), _P, _P, _P, _P]),
    "tessa_sq8_quantize": (TessaStatus, [_P, _U64, _U32, _U32, _U32, _P, _P, _P, _P, _P]),
    "tessa_session_create": (TessaStatus, [C.POINTER(TessaConfig), C.POINTER(_P)]),
    "tessa_session_destroy": (TessaStatus, [_P]),
    "tessa_session_upload_sq8": (TessaStatus, [_P, C.POINTER(Sq8View)]),
    "tessa_session_leaf_topk": (
        TessaStatus,
        [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _P, _P, C.POINTER(C.c_float)],
    ),
    "tessa_session_assign_replay": (
        TessaStatus,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _U32, _P, _P, _P, C.POINTER(C.c_float)],
    ),
    "tessa_plan_subtree": (TessaStatus, [_U64, _U32, _U32, _U32, _U64, _U32, C.POINTER(SubtreePlan)]),
    "tessa_subtree_root_seed": (_U64, [_U64, _U64, _U64, _U64, _U64]),
    "tessa_session_run_subtree": (
        TessaStatus,
        [_P, C.POINTER(SubtreeRequest), C.POINTER(SubtreeOutput)],
    ),
    "tessa_session_partition_roots": (
        TessaStatus,
        [_P, C.POINTER(Sq8View), C.POINTER(RootsRequest), C.POINTER(RootsOutput)],
    ),
    "tessa_session_submit_subtree": (
        TessaStatus,
        [_P, C.POINTER(Sq8View), C.POINTER(SubtreeRequest), C.POINTER(_U64)],
    ),
    "tessa_session_wait": (TessaStatus, [_P, _U64, C.POINTER(SubtreeHostResult)]),
    "tessa_session_release": (TessaStatus, [_P, _U64]),
    "tessa_emit_edge_records": (
        TessaStatus,
        [_P, _U64, C.POINTER(LeafBatch), _P, _P, C.POINTER(SketchView), _P, _U64, _P, C.POINTER(_U64), _P],
    ),
    "tessa_hashprune_create": (TessaStatus, [_U32, _U32, C.POINTER(_P)]),
    "tessa_hashprune_create_backfill": (TessaStatus, [_U32, _U32, C.POINTER(HashPruneBackfill), C.POINTER(_P)]),
    "tessa_hashprune_destroy": (TessaStatus, [_P]),
    "tessa_hashprune_insert": (TessaStatus, [_P, _P, _U64, _P]),
    "tessa_hashprune_neighbors": (TessaStatus, [_P, _P, _P, _P, _P, _P]),
    "tessa_hashprune_clear": (TessaStatus, [_P, _P]),
    "tessa_hashprune_insert_segments": (TessaStatus, [_P, _P, _P, _U64, _P]),
    "tessa_emit_edge_segments": (
        TessaStatus,
        [_P, _U64, C.POINTER(LeafBatch), _P, _P, C.POINTER(SketchView), _P, _U64, _P, _U64, C.POINTER(_U64),
         C.POINTER(_U64), _P],
    ),
    "tessa_emit_edge_segments_unique": (
        TessaStatus,
        [_P, _U64, C.POINTER(LeafBatch), _P, _P, C.POINTER(SketchView), _P, _U64, _P, _U64, C.POINTER(_U64),
         C.POINTER(_U64), _P],
    ),
    "tessa_tierlift_create": (TessaStatus, [C.POINTER(TierLiftConfig), C.POINTER(_P)]),
    "tessa_tierlift_push": (TessaStatus, [_P, _P, _U64, _P, C.POINTER(_U64)]),
    "tessa_tierlift_copied": (TessaStatus, [_P, C.POINTER(_U64)]),
    "tessa_tierlift_wait": (TessaStatus, [_P, _U64]),
    "tessa_tierlift_finish": (TessaStatus, [_P, _P, _P, _P, C.POINTER(TierLiftStats)]),
    "tessa_tierlift_destroy": (TessaStatus, [_P]),
    "tessa_graph_pack": (TessaStatus, [_P, _P, _U32, _U32, _U32, _U64, _P, _U64, C.POINTER(_U64), _P]),
    "tessa_global_d0_assign": (TessaStatus, [_P, _P, _P, _P, _U64, _U32, _P, _P, _P, _P, _U32, _U32, _P, _P, _P, _P, _P]),
    "tessa_robust_prune": (TessaStatus, [_P, _U32, _U32, _P, _P, _U32, _U32, _U32, C.c_float, C.c_int, _P, _P, _P]),
    "tessa_plan_subtree_resident_admission": (TessaStatus, [_U64, _U32, _U32, _U32, _U32, _U64, _U64, _U32, _U32,
                                                             C.POINTER(ResidentAdmission)]),
    "tessa_find_max_admissible_rows": (_U64, [_U32, _U32, _U32, _U32, _U64, _U64, _U32, _U32]),
    "tessa_d0_compute_thresholds": (D0Thresholds, [_U64, C.c_double, C.c_double, C.c_double, _U64]),
    "tessa_d0_plan_root_leaders": (D0LeaderPlan, [_U64, _U64, C.POINTER(D0Thresholds), _U64, _U64]),
    "tessa_d0_split_leader_count": (_U64, [_U64, C.POINTER(D0Thresholds)]),
    "tessa_d0_observe_child_sizes": (D0ChildSummary, [_P, _U64, C.POINTER(D0Thresholds)]),
    "tessa_session_set_assignment_capture": (TessaStatus, [_P, _U32]),
    "tessa_session_captured_assignments": (TessaStatus, [_P, _P, _U64, _P, _U64, C.POINTER(_U64), C.POINTER(_U64)]),
    "tessa_graph_search": (TessaStatus, [_P, _U32, _U32, _P, _P, _U32, _U32, _P, _U32, _U32, _U32, _P, _P, _P, _P]),
    "tessa_graph_search_sq8": (TessaStatus, [_P, _P, _U32, _U32, _U32, _P, _P, _U32, _U32, _P, _U32, _U32, _U32, _P, _P,
                                             _P, _P]),
}

_lib = None


class TessaError(RuntimeError):
    def __init__(self, status: TessaStatus, what: str):
        self.code = int(status.code)
        self.overflow_flags = int(status.overflow_flags)
        self.message = status.msg.decode(errors="replace")
        super().__init__(f"{what}: code={self.code} {self.message}")


def load(path: Path | str | None = None):
    """Load the HIP library once; raises if it is absent (no fallback)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `python -m shear_amd.build` "
            "(the TESSA operator has no CPU fallback)"
        )
    lib = C.CDLL(str(p), mode=getattr(os, "RTLD_NOW", 2) | C.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(status: TessaStatus, what: str) -> None:
    if status.code != TESSA_OK:
        raise TessaError(status, what)


def overflow_labels(flags: int) -> str:
    buf = C.create_string_buffer(256)
    load().tessa_overflow_labels(flags, buf, len(buf))
    return buf.value.decode()


def query_caps(device: int = 0) -> TessaCaps:
    caps = TessaCaps()
    check(load().tessa_query_caps(device, C.byref(caps)), "tessa_query_caps")
    return caps
