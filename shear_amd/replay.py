"""Replay metrics and formal-run contract (host logic of tessa_replay.rs).

Each function restates the named reference function (paths relative to
shear-core/src/algorithm/pipnn/tessa_replay.rs) so replay summaries produced
on MI355X read the same as the reference's.
"""
from __future__ import annotations

import enum
import math
from dataclasses import dataclass
from typing import Sequence


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
    """tessa_replay.rs:211-238 formal contract."""

    seed: int
    warmup_sweeps: int = 5
    measured_sweeps: int = 20
    formal: bool = True

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
