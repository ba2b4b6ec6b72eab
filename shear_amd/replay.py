"""Frozen-task replay of the TESSA operator (host logic of tessa_replay.rs).

Each function restates the named reference function (paths relative to
shear-core/src/algorithm/pipnn/tessa_replay.rs) so replay summaries produced
on MI355X read the same as the reference's.  ``run_tessa_operator_replay``
is the ``tessa_operator_replay run`` command (:333-475): load a capture,
prepare the union rows (:1256-1462), run warmup and measured sweeps of the
modes in rotated order, check the exact (DP4A role) and MFMA (WMMA role)
executors bit for bit and every mode's determinism across measured sweeps,
and write samples.tsv, task_metrics.tsv, summary.json and summary.md
(create-new).  This build has no fp32 / TF32 leaf backends, so it runs the
four SQ8 modes (A2, A3 and the two SQ8 auxiliaries); the overlap metrics use
A2, the exact executor, where the reference uses A0.
"""
from __future__ import annotations

import ctypes as C
import enum
import json
import math
import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import Sequence

import numpy as np


class TessaReplayMode(enum.Enum):
    """tessa_replay.rs:20-86 (the SQ8 modes are the ones this build runs)."""

    A0_FP32_SIMT = "a0-fp32-simt"
    A1_TF32_WMMA = "a1-tf32-wmma"
    A2_SQ8_DP4A_BATCH1 = "a2-sq8-dp4a-batch1"
    A3_SQ8_WMMA_BATCH8 = "a3-sq8-wmma-batch8"
    SQ8_DP4A_BATCH8 = "sq8-dp4a-batch8"
    SQ8_WMMA_BATCH1 = "sq8-wmma-batch1"

    @property
    def uses_sq8(self) -> bool:
        return self not in (TessaReplayMode.A0_FP32_SIMT, TessaReplayMode.A1_TF32_WMMA)

    @property
    def replays_leaf_tasks(self) -> bool:
        return self in (TessaReplayMode.A0_FP32_SIMT, TessaReplayMode.A1_TF32_WMMA,
                        TessaReplayMode.A2_SQ8_DP4A_BATCH1, TessaReplayMode.A3_SQ8_WMMA_BATCH8)

    @property
    def assignment_ticket_batch(self) -> int:
        return 8 if self in (TessaReplayMode.A3_SQ8_WMMA_BATCH8, TessaReplayMode.SQ8_DP4A_BATCH8) else 1

    @property
    def leaf_executor_code(self) -> int | None:
        """0 fp32, 1 exact scalar (DP4A role), 2 matrix cores (WMMA role)."""
        return {
            TessaReplayMode.A0_FP32_SIMT: 0,
            TessaReplayMode.A1_TF32_WMMA: 0,
            TessaReplayMode.A2_SQ8_DP4A_BATCH1: 1,
            TessaReplayMode.A3_SQ8_WMMA_BATCH8: 2,
        }.get(self)


ALL_MODES = list(TessaReplayMode)


def tessa_rotated_mode_order(sweep: int) -> list[TessaReplayMode]:
    """tessa_replay.rs:1245-1250."""
    r = sweep % len(ALL_MODES)
    return ALL_MODES[r:] + ALL_MODES[:r]


@dataclass(frozen=True)
class TessaCandidateBlock:
    output_offset: int
    rows: int
    width: int
    pair_weight: int


@dataclass(frozen=True)
class TessaOverlapSummary:
    task_count: int = 0
    macro_mean: float = 0.0
    pair_weighted_mean: float = 0.0
    p5: float = 0.0
    p50: float = 0.0
    p95: float = 0.0
    exact_task_fraction: float = 0.0


@dataclass(frozen=True)
class TessaDistributionSummary:
    median: float
    min: float
    max: float


@dataclass(frozen=True)
class TessaReplayRunConfig:
    """tessa_replay.rs:211-238 formal contract (the paths are those of the
    replay command; the metric helpers only read the sweep counts)."""

    seed: int
    warmup_sweeps: int = 5
    measured_sweeps: int = 20
    formal: bool = True
    manifest_path: str = ""
    base_path: str = ""
    output_dir: str = ""
    gpu_device: int = 0

    def validate(self) -> None:
        if self.formal and (self.warmup_sweeps != 5 or self.measured_sweeps != 20):
            raise ValueError(f"formal replay requires exactly 5 warmup and 20 measured sweeps, "
                             f"got {self.warmup_sweeps}/{self.measured_sweeps}")
        if self.warmup_sweeps == 0 or self.measured_sweeps == 0:
            raise ValueError("warmup_sweeps and measured_sweeps must both be positive")
        if self.seed == 0:
            raise ValueError("replay seed must be non-zero")


def tessa_assignment_pairs(tasks: Sequence[tuple[int, int]]) -> int:
    """tessa_replay.rs:1059-1074; tasks as (member_count, leader_count)."""
    return sum(m * l for m, l in tasks)


def tessa_leaf_pairs(member_counts: Sequence[int]) -> int:
    """tessa_replay.rs:1076-1087: sum of n*(n-1)."""
    return sum(n * max(n - 1, 0) for n in member_counts)


def _logical_payload_bytes(unique_rows: int, dims: int, bytes_per_dim: int, meta: int) -> int:
    return unique_rows * (dims * bytes_per_dim + meta)


def tessa_fp32_logical_payload_bytes(unique_rows: int, dim: int) -> int:
    """tessa_replay.rs:1089-1091."""
    return _logical_payload_bytes(unique_rows, dim, 4, 4)


def tessa_sq8_logical_payload_bytes(unique_rows: int, padded_dim: int) -> int:
    """tessa_replay.rs:1093-1095: codes plus scale and norm per row."""
    return _logical_payload_bytes(unique_rows, padded_dim, 1, 8)


def tessa_nearest_rank_percentile(values: Sequence[float], percentile: float) -> float:
    """tessa_replay.rs:1112-1127."""
    if not values:
        raise ValueError("percentile requires at least one value")
    if not math.isfinite(percentile) or not 0.0 <= percentile <= 1.0:
        raise ValueError("percentile must be finite and in [0, 1]")
    if any(not math.isfinite(v) for v in values):
        raise ValueError("percentile input contains a non-finite value")
    s = sorted(values)
    rank = math.ceil(percentile * len(s))
    return s[min(max(rank, 1), len(s)) - 1]


def tessa_distribution_summary(values: Sequence[float]) -> TessaDistributionSummary:
    """tessa_replay.rs:1129-1150."""
    if not values:
        raise ValueError("distribution summary requires at least one value")
    if any(not math.isfinite(v) for v in values):
        raise ValueError("distribution summary input contains a non-finite value")
    s = sorted(values)
    mid = len(s) // 2
    median = (s[mid - 1] + s[mid]) / 2.0 if len(s) % 2 == 0 else s[mid]
    return TessaDistributionSummary(median, s[0], s[-1])


def tessa_overlap_summary(reference_ids, actual_ids, blocks: Sequence[TessaCandidateBlock]) -> TessaOverlapSummary:
    """tessa_replay.rs:1152-1226: per-block fraction of reference ids present in
    the actual row (EMPTY ids ignored), macro and pair-weighted means,
    nearest-rank p5/p50/p95 and the fraction of blocks that match exactly."""
    ref = list(reference_ids)
    act = list(actual_ids)
    if len(ref) != len(act):
        raise ValueError(f"candidate output length mismatch: reference={len(ref)} actual={len(act)}")
    if not blocks:
        return TessaOverlapSummary()
    empty = 0xFFFFFFFF
    overlaps, wsum, wtot, exact = [], 0.0, 0, 0
    for b in blocks:
        if b.width == 0:
            raise ValueError("candidate block width must be positive")
        n = b.rows * b.width
        end = b.output_offset + n
        if end > len(ref):
            raise ValueError(f"candidate block {b.output_offset}..{end} exceeds output length {len(ref)}")
        r = ref[b.output_offset:end]
        a = act[b.output_offset:end]
        matches = 0
        for i in range(0, n, b.width):
            aset = {x for x in a[i:i + b.width] if x != empty}
            matches += sum(1 for x in r[i:i + b.width] if x != empty and x in aset)
        ov = 1.0 if n == 0 else matches / n
        overlaps.append(ov)
        wsum += ov * b.pair_weight
        wtot += b.pair_weight
        exact += int(r == a)
    return TessaOverlapSummary(
        task_count=len(blocks),
        macro_mean=sum(overlaps) / len(overlaps),
        pair_weighted_mean=0.0 if wtot == 0 else wsum / wtot,
        p5=tessa_nearest_rank_percentile(overlaps, 0.05),
        p50=tessa_nearest_rank_percentile(overlaps, 0.50),
        p95=tessa_nearest_rank_percentile(overlaps, 0.95),
        exact_task_fraction=exact / len(blocks),
    )


# ---- the replay command ----------------------------------------------------

RUN_MODES = [m for m in ALL_MODES if m.uses_sq8]  # the modes this build runs
OVERLAP_REFERENCE = TessaReplayMode.A2_SQ8_DP4A_BATCH1
OUTPUT_FILES = ("samples.tsv", "task_metrics.tsv", "summary.json", "summary.md", "failure.json")
MISMATCH_SAMPLE_LIMIT = 64


class ReplayError(RuntimeError):
    """tessa_replay.rs:1457-1459 replay_error: messages start with 'TESSA replay: '."""

    def __init__(self, msg: str):
        super().__init__(f"TESSA replay: {msg}")


def rotated_run_modes(sweep: int) -> list[TessaReplayMode]:
    """tessa_rotated_mode_order over the modes this build runs."""
    r = sweep % len(RUN_MODES)
    return RUN_MODES[r:] + RUN_MODES[:r]


@dataclass
class PreparedReplay:
    """TessaPreparedReplay (tessa_replay.rs:1047-1057)."""

    dim: int
    padded_dim: int
    global_ids: np.ndarray          # u32 union of the tasks' rows, ascending
    sq8: object                     # tessa.Sq8Matrix of the union rows (device)
    assignment_members: np.ndarray  # local rows
    assignment_leaders: np.ndarray
    assignment_layouts: list        # (member_offset, member_count, leader_offset, leader_count, r_h, output_offset)
    leaf_members: np.ndarray
    leaf_layouts: list              # (member_offset, member_count, k, output_offset)
    leaf_k: int
    assignment_blocks: list
    leaf_blocks: list
    assignment_pairs: int
    leaf_pairs: int
    assignment_unique_rows: int
    leaf_unique_rows: int


def read_fbin_rows(path, rows: np.ndarray) -> np.ndarray:
    """Rows of an .fbin file (u32 rows, u32 dim, then rows x dim f32), in the given order."""
    with open(path, "rb") as f:
        n, dim = np.frombuffer(f.read(8), "<u4")
    data = np.memmap(path, dtype="<f4", mode="r", offset=8, shape=(int(n), int(dim)))
    return np.ascontiguousarray(data[np.asarray(rows, np.int64)], np.float32)


def prepare_tessa_replay(manifest: dict, selection, base_path, device="cuda") -> PreparedReplay:
    """tessa_replay.rs:1256-1462: union rows, SQ8 payload, layouts and blocks."""
    import torch

    from . import tessa as T

    with open(base_path, "rb") as f:
        n, dim = (int(v) for v in np.frombuffer(f.read(8), "<u4"))
    if n != manifest["dataset"]["rows"] or dim != manifest["dataset"]["dimension"]:
        raise ReplayError(f"base shape mismatch: base={n}x{dim} capture="
                          f"{manifest['dataset']['rows']}x{manifest['dataset']['dimension']}")
    a_ids = {i for t in selection.assignment_tasks for i in list(t.member_ids) + list(t.leader_ids)}
    l_ids = {i for t in selection.leaf_tasks for i in t.member_ids}
    gids = np.array(sorted(a_ids | l_ids), np.uint32)
    if len(gids) == 0:
        raise ReplayError("capture contains no replay rows")
    x = read_fbin_rows(base_path, gids)
    sq8 = T.quantize_sq_int8_matrix(torch.from_numpy(x).to(device))
    local = {int(g): i for i, g in enumerate(gids.tolist())}

    def mapped(ids):
        try:
            return [local[int(i)] for i in ids]
        except KeyError as e:
            raise ReplayError(f"captured global row {e.args[0]} is missing from replay union") from None

    am, al, alay, ablk, off = [], [], [], [], 0
    for t in selection.assignment_tasks:
        if t.padded_dim != sq8.padded_dim:
            raise ReplayError(f"assignment task padded_dim mismatch: captured={t.padded_dim} "
                              f"prepared={sq8.padded_dim}")
        if t.r_h == 0 or t.r_h > 4 or t.r_h > len(t.leader_ids):
            raise ReplayError(f"assignment task {t.task_hash} has invalid r_h={t.r_h} for "
                              f"{len(t.leader_ids)} leaders")
        alay.append((len(am), len(t.member_ids), len(al), len(t.leader_ids), t.r_h, off))
        ablk.append(TessaCandidateBlock(off, len(t.member_ids), t.r_h, len(t.member_ids) * len(t.leader_ids)))
        am += mapped(t.member_ids)
        al += mapped(t.leader_ids)
        off += len(t.member_ids) * t.r_h
    lm, llay, lblk, off, k = [], [], [], 0, None
    for t in selection.leaf_tasks:
        if t.padded_dim != sq8.padded_dim:
            raise ReplayError(f"leaf task padded_dim mismatch: captured={t.padded_dim} prepared={sq8.padded_dim}")
        if t.k == 0 or t.k >= len(t.member_ids):
            raise ReplayError(f"leaf task {t.task_hash} has invalid k={t.k} for {len(t.member_ids)} rows")
        if k is not None and k != t.k:
            raise ReplayError(f"captured leaf tasks must use one k, found {k} and {t.k}")
        k = t.k
        llay.append((len(lm), len(t.member_ids), t.k, off))
        n_ = len(t.member_ids)
        lblk.append(TessaCandidateBlock(off, n_, t.k, n_ * (n_ - 1)))
        lm += mapped(t.member_ids)
        off += n_ * t.k
    if k is None:
        raise ReplayError("capture contains no leaf tasks")
    if not alay:
        raise ReplayError("capture contains no assignment tasks")
    return PreparedReplay(dim, sq8.padded_dim, gids, sq8, np.array(am, np.uint32), np.array(al, np.uint32), alay,
                          np.array(lm, np.uint32), llay, k, ablk, lblk,
                          tessa_assignment_pairs([(len(t.member_ids), len(t.leader_ids))
                                                  for t in selection.assignment_tasks]),
                          tessa_leaf_pairs([len(t.member_ids) for t in selection.leaf_tasks]),
                          len(a_ids), len(l_ids))


@dataclass
class ModeResult:
    """TessaCudaModeResult (tessa_replay.rs:190-200)."""

    assignment_event_ms: float
    leaf_event_ms: float | None
    total_event_ms: float
    assignment_ids: np.ndarray
    assignment_dists: np.ndarray
    leaf_ids: np.ndarray
    leaf_dists: np.ndarray
    counters: dict = field(default_factory=dict)


def _replay_counters(leaf_ctr: np.ndarray, assign_ctr: np.ndarray, leaf_exec: int | None) -> dict:
    """TessaCudaReplayCounters (tessa_replay.rs:154-176) from the library's
    counter words; words with no counterpart here (watchdog, queue heads,
    ticket claims) are 0."""
    from . import _native as N

    lc = leaf_ctr if leaf_ctr is not None else np.zeros(N.COUNTER_WORDS, np.uint64)
    return {"overflow_flags": int(lc[N.C_OVERFLOW_FLAGS]) | int(assign_ctr[N.C_OVERFLOW_FLAGS]),
            "watchdog_trips": 0, "assignment_fallback_nodes": 0, "assignment_overflow_nodes": 0,
            "leaf_exact_fallback_rows": int(lc[N.C_LEAF_FALLBACK_ROWS]),
            "leaf_survivor_overflow_rows": int(lc[N.C_LEAF_LIST_OVERFLOW_ROWS]),
            "large_split_retries": 0, "large_balanced_fallbacks": 0, "assignment_ticket_claims": 0,
            "assignment_physical_tiles": 0, "assignment_dp4a_tiles": 0,
            "assignment_wmma_tiles": int(assign_ctr[N.C_ASSIGN_ROWS]),
            "leaf_dp4a_tiles": int(lc[N.C_LEAF_EXACT_ROWS]) if leaf_exec == N.EXEC_EXACT else 0,
            "leaf_wmma_tiles": int(lc[N.C_LEAF_MFMA_TILES]) if leaf_exec == N.EXEC_MFMA else 0,
            "leaf_head": 0, "leaf_pushes": 0, "leaf_topk_pops": 0, "leaf_col_tasks_started": 0,
            "leaf_col_tasks_done": 0, "leaf_finalize_started": 0, "leaf_finalize_done": 0}


def fallback_count(c: dict) -> int:
    """tessa_replay.rs:179-187."""
    return (c["assignment_fallback_nodes"] + c["assignment_overflow_nodes"] + c["leaf_exact_fallback_rows"]
            + c["leaf_survivor_overflow_rows"] + c["large_split_retries"] + c["large_balanced_fallbacks"])


class ReplaySession:
    """TessaCudaReplaySession (compute_backend.rs:34590-35324) over the C ABI:
    the prepared union rows resident on one device, one mode per call."""

    def __init__(self, device: int, prep: PreparedReplay):
        from . import _native as N
        from . import tessa as T

        self._N = N
        self._lib = N.load()
        h = C.c_void_p()
        N.check(self._lib.tessa_session_create(C.byref(N.TessaConfig(device, 0)), C.byref(h)), "session create")
        self._h = h
        gids = np.ascontiguousarray(prep.global_ids, np.uint32)
        import torch

        g = torch.from_numpy(gids.view(np.int32)).to(prep.sq8.codes.device)
        view = prep.sq8.view(g)
        torch.cuda.synchronize()
        N.check(self._lib.tessa_session_upload_sq8(self._h, C.byref(view)), "session upload")
        self.prep = prep
        a = prep.assignment_layouts
        self._a = [np.ascontiguousarray(v) for v in (
            prep.assignment_members, prep.assignment_leaders, np.array([t[0] for t in a], np.uint32),
            np.array([t[1] for t in a], np.uint32), np.array([t[2] for t in a], np.uint32),
            np.array([t[3] for t in a], np.uint32), np.array([t[4] for t in a], np.uint32),
            np.array([t[5] for t in a], np.uint64))]
        self._a_len = sum(t[1] * t[4] for t in a)
        lay = prep.leaf_layouts
        self._l = [np.ascontiguousarray(v) for v in (
            prep.leaf_members, np.array([t[0] for t in lay], np.uint64), np.array([t[1] for t in lay], np.uint32),
            np.array([t[3] for t in lay], np.uint64))]
        self._l_len = sum(t[1] * t[2] for t in lay)

    def close(self):
        if self._h:
            self._N.check(self._lib.tessa_session_destroy(self._h), "session destroy")
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run_mode(self, mode: TessaReplayMode) -> ModeResult:
        N = self._N
        p = self.prep
        a_ids = np.zeros(max(self._a_len, 1), np.uint32)
        a_d = np.zeros(max(self._a_len, 1), np.float32)
        a_ctr = np.zeros(N.COUNTER_WORDS, np.uint64)
        a_ms = C.c_float(0.0)
        am, al, mo, mc, lo, lc, rh, oo = self._a
        N.check(self._lib.tessa_session_assign_replay(
            self._h, am.ctypes.data, al.ctypes.data, mo.ctypes.data, mc.ctypes.data, lo.ctypes.data, lc.ctypes.data,
            rh.ctypes.data, oo.ctypes.data, len(p.assignment_layouts), a_ids.ctypes.data, a_d.ctypes.data,
            a_ctr.ctypes.data, C.byref(a_ms)), f"replay {mode.value} assignment")
        leaf_ms = None
        l_ids = np.zeros(0, np.uint32)
        l_d = np.zeros(0, np.float32)
        l_ctr = None
        exe = mode.leaf_executor_code
        if mode.replays_leaf_tasks:
            l_ids = np.zeros(max(self._l_len, 1), np.uint32)
            l_d = np.zeros(max(self._l_len, 1), np.float32)
            l_ctr = np.zeros(N.COUNTER_WORDS, np.uint64)
            ms = C.c_float(0.0)
            lm, lof, lcn, loo = self._l
            N.check(self._lib.tessa_session_leaf_topk(
                self._h, lm.ctypes.data, lof.ctypes.data, lcn.ctypes.data, loo.ctypes.data, len(p.leaf_layouts),
                p.leaf_k, exe, l_ids.ctypes.data, l_d.ctypes.data, l_ctr.ctypes.data, C.byref(ms)),
                f"replay {mode.value} leaf")
            leaf_ms = float(ms.value)
            l_ids, l_d = l_ids[: self._l_len], l_d[: self._l_len]
        a_ids, a_d = a_ids[: self._a_len], a_d[: self._a_len]
        total = float(a_ms.value) + (leaf_ms or 0.0)
        return ModeResult(float(a_ms.value), leaf_ms, total, a_ids, a_d, l_ids, l_d,
                          _replay_counters(l_ctr, a_ctr, exe))


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return len(a) == len(b) and np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                                               np.asarray(b, np.float32).view(np.uint32))


def candidate_mismatch_detail(kind, ids_a, d_a, ids_b, d_b, blocks):
    """tessa_replay.rs:631-737 (A2 as 'dp4a', A3 as 'wmma')."""
    ia, ib = np.asarray(ids_a, np.uint32), np.asarray(ids_b, np.uint32)
    da, db = np.asarray(d_a, np.float32).view(np.uint32), np.asarray(d_b, np.float32).view(np.uint32)
    m = min(len(ia), len(ib))
    md = min(len(da), len(db))
    id_mis = int(np.count_nonzero(ia[:m] != ib[:m])) + abs(len(ia) - len(ib))
    d_mis = int(np.count_nonzero(da[:md] != db[:md])) + abs(len(da) - len(db))
    if id_mis == 0 and d_mis == 0:
        return None
    n = max(len(ia), len(ib), len(da), len(db))

    def get(a, i):
        return int(a[i]) if i < len(a) else None

    idx = [i for i in range(n) if get(ia, i) != get(ib, i) or get(da, i) != get(db, i)]
    samples = []
    for i in idx[:MISMATCH_SAMPLE_LIMIT]:
        loc = None
        for ti, b in enumerate(blocks):
            if b.width and b.output_offset <= i < b.output_offset + b.rows * b.width:
                li = i - b.output_offset
                loc = (ti, li // b.width, li % b.width, b)
                break
        samples.append({"index": i, "task_index": loc[0] if loc else None, "row": loc[1] if loc else None,
                        "rank": loc[2] if loc else None, "block_rows": loc[3].rows if loc else None,
                        "block_width": loc[3].width if loc else None,
                        "block_pair_weight": loc[3].pair_weight if loc else None,
                        "dp4a_id": get(ia, i), "wmma_id": get(ib, i), "dp4a_distance_bits": get(da, i),
                        "wmma_distance_bits": get(db, i)})
    first = samples[0]
    out = {"kind": kind, "dp4a_id_len": len(ia), "wmma_id_len": len(ib), "dp4a_distance_len": len(da),
           "wmma_distance_len": len(db), "id_mismatch_count": id_mis, "distance_bit_mismatch_count": d_mis,
           "mismatch_index_count": len(idx), "mismatch_sample_limit": MISMATCH_SAMPLE_LIMIT,
           "mismatch_sample_truncated": len(idx) > len(samples), "mismatches": samples,
           "first_index": first["index"]}
    out.update({k: first[k] for k in ("task_index", "row", "rank", "block_rows", "block_width", "block_pair_weight",
                                      "dp4a_id", "wmma_id", "dp4a_distance_bits", "wmma_distance_bits")})
    return out


def _write_new(path: Path, data: bytes) -> None:
    """tessa_replay.rs:1015-1027: create-new, then sync."""
    fd = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    with os.fdopen(fd, "wb") as f:
        f.write(data)
        f.flush()
        os.fsync(f.fileno())


def samples_tsv(samples: list) -> str:
    """tessa_replay.rs:786-828."""
    out = ["phase\tsweep\torder\tmode\ttask_kind\tevent_ms\tpairs\tthroughput_pairs_per_s\tlogical_payload_bytes"
           "\toverflow_flags\tfallback_count\twatchdog_trips\tticket_claims\tphysical_tiles"
           "\tassignment_dp4a_tiles\tassignment_wmma_tiles\tleaf_dp4a_tiles\tleaf_wmma_tiles\n"]
    for s in samples:
        c = s["counters"]
        thr = s["pairs"] * 1000.0 / s["event_ms"] if s["event_ms"] > 0 else 0.0
        out.append(f"{s['phase']}\t{s['sweep']}\t{s['order']}\t{s['mode']}\t{s['kind']}\t{s['event_ms']:.9f}\t"
                   f"{s['pairs']}\t{thr:.6f}\t{s['payload']}\t{c['overflow_flags']}\t{fallback_count(c)}\t"
                   f"{c['watchdog_trips']}\t{c['assignment_ticket_claims']}\t{c['assignment_physical_tiles']}\t"
                   f"{c['assignment_dp4a_tiles']}\t{c['assignment_wmma_tiles']}\t{c['leaf_dp4a_tiles']}\t"
                   f"{c['leaf_wmma_tiles']}\n")
    return "".join(out)


def task_metrics_tsv(canonical: dict, prep: PreparedReplay) -> str:
    """tessa_replay.rs:830-886, with A2 as the overlap reference."""
    ref = canonical[OVERLAP_REFERENCE]
    out = ["mode\ttask_kind\ttask_index\tpair_weight\toverlap\texact\n"]
    for mode in RUN_MODES:
        act = canonical[mode]
        kinds = [("assignment", ref.assignment_ids, act.assignment_ids, prep.assignment_blocks)]
        if mode.replays_leaf_tasks:
            kinds.append(("leaf", ref.leaf_ids, act.leaf_ids, prep.leaf_blocks))
        for kind, r, a, blocks in kinds:
            for ti, b in enumerate(blocks):
                ov = tessa_overlap_summary(r, a, [b]).macro_mean
                end = b.output_offset + b.rows * b.width
                exact = int(np.array_equal(r[b.output_offset:end], a[b.output_offset:end]))
                out.append(f"{mode.value}\t{kind}\t{ti}\t{b.pair_weight}\t{ov:.9f}\t{exact}\n")
    return "".join(out)


def _dist(values):
    d = tessa_distribution_summary(values)
    return {"median": d.median, "min": d.min, "max": d.max}


def _overlap(o: TessaOverlapSummary):
    return {"task_count": o.task_count, "macro_mean": o.macro_mean, "pair_weighted_mean": o.pair_weighted_mean,
            "p5": o.p5, "p50": o.p50, "p95": o.p95, "exact_task_fraction": o.exact_task_fraction}


def summary_json(cfg: TessaReplayRunConfig, manifest: dict, prep: PreparedReplay, samples: list,
                 canonical: dict) -> dict:
    """tessa_replay.rs:888-954."""
    ref = canonical[OVERLAP_REFERENCE]
    modes = []
    for mode in RUN_MODES:
        act = canonical[mode]

        def measured(kind):
            return [s["event_ms"] for s in samples if s["phase"] == "measured" and s["mode"] == mode.value
                    and s["kind"] == kind]

        a_ms, t_ms, l_ms = measured("assignment"), measured("total"), measured("leaf")
        ad, td = _dist(a_ms), _dist(t_ms)
        ld = _dist(l_ms) if l_ms else None
        modes.append({
            "mode": mode.value,
            "assignment_event_ms": ad, "leaf_event_ms": ld, "total_event_ms": td,
            "assignment_throughput_pairs_per_s": prep.assignment_pairs * 1000.0 / ad["median"] if ad["median"] else 0.0,
            "leaf_throughput_pairs_per_s": (prep.leaf_pairs * 1000.0 / ld["median"]) if ld and ld["median"] else None,
            "assignment_logical_payload_bytes": tessa_sq8_logical_payload_bytes(prep.assignment_unique_rows,
                                                                                prep.padded_dim),
            "leaf_logical_payload_bytes": (tessa_sq8_logical_payload_bytes(prep.leaf_unique_rows, prep.padded_dim)
                                           if mode.replays_leaf_tasks else None),
            "assignment_overlap_at_rh": _overlap(tessa_overlap_summary(ref.assignment_ids, act.assignment_ids,
                                                                       prep.assignment_blocks)),
            "leaf_overlap_at_k": (_overlap(tessa_overlap_summary(ref.leaf_ids, act.leaf_ids, prep.leaf_blocks))
                                  if mode.replays_leaf_tasks else None),
            "safety_counters": act.counters,
        })
    return {"schema_version": 1, "formal": cfg.formal, "seed": cfg.seed, "warmup_sweeps": cfg.warmup_sweeps,
            "measured_sweeps": cfg.measured_sweeps, "gpu_device": cfg.gpu_device, "capture_manifest": manifest,
            "assignment_pairs": prep.assignment_pairs, "leaf_pairs": prep.leaf_pairs,
            "overlap_reference_mode": OVERLAP_REFERENCE.value,
            "a2_a3_candidate_ids_and_distance_bits_exact": True, "modes": modes}


def summary_markdown(summary: dict) -> str:
    """tessa_replay.rs:970-1013."""
    out = ["# TESSA operator replay\n\n| Mode | Assignment ms (median [min, max]) | Leaf ms | Total ms | "
           "Assignment overlap | Leaf overlap |\n|---|---:|---:|---:|---:|---:|\n"]
    for m in summary["modes"]:
        def dist(key):
            v = m[key]
            return "N/A" if v is None else f"{v['median']:.3f} [{v['min']:.3f}, {v['max']:.3f}]"

        lo = m["leaf_overlap_at_k"]
        out.append(f"| {m['mode']} | {dist('assignment_event_ms')} | {dist('leaf_event_ms')} | "
                   f"{dist('total_event_ms')} | {m['assignment_overlap_at_rh']['macro_mean']:.6f} | "
                   f"{'N/A' if lo is None else format(lo['macro_mean'], '.6f')} |\n")
    out.append("\nA2 and A3 candidate IDs and `f32` distance bits are exactly identical.\n")
    return "".join(out)


def run_tessa_operator_replay(cfg: TessaReplayRunConfig) -> Path:
    """tessa_replay.rs:333-475 (+ :380-475 for the run itself); returns the
    output directory.  Raises ReplayError on any contract violation, after
    writing failure.json when A2 and A3 differ."""
    from . import capture as CP

    cfg.validate()
    mp = Path(cfg.manifest_path)
    if mp.is_dir():
        cap_dir = mp
    elif mp.name == CP.MANIFEST_FILE:
        cap_dir = mp.parent
    else:
        raise ReplayError(f"manifest must name {CP.MANIFEST_FILE} or its containing directory, got {mp}")
    manifest, selection = CP.load_tessa_capture(cap_dir, CP.dataset_metadata(cfg.base_path))
    if manifest["provenance"]["seed"] != cfg.seed:
        raise ReplayError(f"replay seed mismatch: requested={cfg.seed} captured={manifest['provenance']['seed']}")
    prep = prepare_tessa_replay(manifest, selection, cfg.base_path)
    out_dir = Path(cfg.output_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    for f in OUTPUT_FILES:
        if (out_dir / f).exists():
            raise ReplayError(f"refusing to overwrite replay output {out_dir / f}")
    sess = ReplaySession(cfg.gpu_device, prep)
    samples, canonical = [], {}
    try:
        for phase, count in (("warmup", cfg.warmup_sweeps), ("measured", cfg.measured_sweeps)):
            for sweep in range(count):
                results = {}
                for order, mode in enumerate(rotated_run_modes(sweep)):
                    r = sess.run_mode(mode)
                    a_pay = tessa_sq8_logical_payload_bytes(prep.assignment_unique_rows, prep.padded_dim)
                    samples.append({"phase": phase, "sweep": sweep, "order": order, "mode": mode.value,
                                    "kind": "assignment", "event_ms": r.assignment_event_ms,
                                    "pairs": prep.assignment_pairs, "payload": a_pay, "counters": r.counters})
                    tp, tpay = prep.assignment_pairs, a_pay
                    if r.leaf_event_ms is not None:
                        l_pay = tessa_sq8_logical_payload_bytes(prep.leaf_unique_rows, prep.padded_dim)
                        samples.append({"phase": phase, "sweep": sweep, "order": order, "mode": mode.value,
                                        "kind": "leaf", "event_ms": r.leaf_event_ms, "pairs": prep.leaf_pairs,
                                        "payload": l_pay, "counters": r.counters})
                        tp, tpay = tp + prep.leaf_pairs, tpay + l_pay
                    samples.append({"phase": phase, "sweep": sweep, "order": order, "mode": mode.value,
                                    "kind": "total", "event_ms": r.total_event_ms, "pairs": tp, "payload": tpay,
                                    "counters": r.counters})
                    if phase == "measured":
                        e = canonical.get(mode)
                        if e is None:
                            canonical[mode] = r
                        elif not (np.array_equal(e.assignment_ids, r.assignment_ids)
                                  and np.array_equal(e.leaf_ids, r.leaf_ids)
                                  and _same_bits(e.assignment_dists, r.assignment_dists)
                                  and _same_bits(e.leaf_dists, r.leaf_dists)):
                            raise ReplayError(f"mode {mode.value} produced non-deterministic candidate output "
                                              f"across measured sweeps")
                    results[mode] = r
                a2, a3 = results[TessaReplayMode.A2_SQ8_DP4A_BATCH1], results[TessaReplayMode.A3_SQ8_WMMA_BATCH8]
                am = candidate_mismatch_detail("assignment", a2.assignment_ids, a2.assignment_dists,
                                               a3.assignment_ids, a3.assignment_dists, prep.assignment_blocks)
                lm = candidate_mismatch_detail("leaf", a2.leaf_ids, a2.leaf_dists, a3.leaf_ids, a3.leaf_dists,
                                               prep.leaf_blocks)
                if am or lm:
                    fail = {"schema_version": 2,
                            "message": "A2 SQ8-DP4A and A3 SQ8-WMMA candidate IDs or distance bits differ",
                            "phase": phase, "sweep": sweep, "dp4a_counters": a2.counters,
                            "wmma_counters": a3.counters, "assignment": am, "leaf": lm}
                    _write_new(out_dir / "failure.json", (json.dumps(fail, indent=2) + "\n").encode())
                    kinds = " and ".join(k for k, v in (("assignment", am), ("leaf", lm)) if v)
                    raise ReplayError(f"A2 SQ8-DP4A and A3 SQ8-WMMA {kinds} candidate output differs; "
                                      f"details: {out_dir / 'failure.json'}")
    finally:
        sess.close()
    summary = summary_json(cfg, manifest, prep, samples, canonical)
    _write_new(out_dir / "samples.tsv", samples_tsv(samples).encode())
    _write_new(out_dir / "task_metrics.tsv", task_metrics_tsv(canonical, prep).encode())
    _write_new(out_dir / "summary.json", (json.dumps(summary, indent=2) + "\n").encode())
    _write_new(out_dir / "summary.md", summary_markdown(summary).encode())
    return out_dir


def main(argv=None) -> int:
    """``python -m shear_amd.replay run --manifest M --base B --output-dir O --seed S``
    (apps/tessa_operator_replay/src/main.rs:16-65 ``run``)."""
    import argparse

    ap = argparse.ArgumentParser(prog="tessa_operator_replay")
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--manifest", required=True)
    r.add_argument("--base", required=True)
    r.add_argument("--output-dir", required=True)
    r.add_argument("--gpu-device", type=int, default=0)
    r.add_argument("--seed", type=int, required=True)
    r.add_argument("--warmup-sweeps", type=int, default=5)
    r.add_argument("--measured-sweeps", type=int, default=20)
    r.add_argument("--formal", action="store_true")
    a = ap.parse_args(argv)
    out = run_tessa_operator_replay(TessaReplayRunConfig(
        seed=a.seed, warmup_sweeps=a.warmup_sweeps, measured_sweeps=a.measured_sweeps, formal=a.formal,
        manifest_path=a.manifest, base_path=a.base, output_dir=a.output_dir, gpu_device=a.gpu_device))
    print(f"replay written to {out}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
