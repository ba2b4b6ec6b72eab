"""Global D0 assignment: the task formation above the GPU subtrees.

Host mirror of the reference's D0 level (paths relative to
shear-core/src/algorithm/pipnn/):

* ``adaptive_psamp_fraction``   params.rs:2977-3001 (leader sampling rate by size and depth)
* ``d0_leader_count``           leaders of a node of n points: min(n * rate, max_leaders)
                                (params.rs:3258-3262)
* ``D0CapacityConfig`` / ``compute_thresholds`` / ``plan_root_leaders`` /
  ``split_leader_count`` / ``observe_child_unique_sizes``   d0_capacity.rs:1-299
  (libtessa_hip.so ``tessa_d0_*``)
* ``find_max_admissible_rows``  d0_capacity.rs:55-102 over the resident admission plan
                                (compute_backend.rs:1490-1522; ``tessa_find_max_admissible_rows``)
* ``global_d0_assign``          the GPU-D0 SQ8 assignment (compute_backend.rs:18016-18511;
                                CPU statement dco_sq_int8.rs:1929-2064): each row to its
                                fanout_top nearest leaders, fragments grouped into the D0
                                children.  Runs in libtessa_hip.so (``tessa_global_d0_assign``).

The reference samples the D0 leaders with rand's StdRng
(rbc_partition.rs); that stream is not reproducible here, so callers pass
the leader rows (``sample_leader_rows`` draws them with a seeded torch
generator).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N
from .tessa import Sq8Matrix, _ptr, _stream_ptr


def adaptive_psamp_fraction(psamp_fraction: float, cluster_size: int, depth: int) -> float:
    frac = psamp_fraction
    for limit, mul in ((20_000_000, 0.05), (10_000_000, 0.1), (5_000_000, 0.2), (1_000_000, 0.4), (100_000, 0.7)):
        if cluster_size >= limit:
            frac *= mul
            break
    if depth > 4:
        frac *= 0.35
    elif depth > 2:
        frac *= 0.5
    elif depth > 0:
        frac *= 0.8
    return min(max(frac, 0.00005), 0.1)


def d0_leader_count(n: int, psamp_fraction: float = 0.001, max_leaders: int = 1000) -> int:
    return max(1, int(min(n * adaptive_psamp_fraction(psamp_fraction, n, 0), max_leaders)))


def sample_leader_rows(n: int, count: int, seed: int, device="cuda") -> torch.Tensor:
    """``count`` distinct rows of [0, n), ascending (int64)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return torch.randperm(n, generator=g)[:count].sort().values.to(device)


def global_d0_assign(sq8: Sq8Matrix, global_ids: torch.Tensor, leaders: Sq8Matrix, leader_ids: torch.Tensor,
                     fanout_top: int = 10, group: bool = True, stream: torch.cuda.Stream | None = None):
    """(child int32 [rows, fanout], point int32 [rows, fanout], child_offsets
    int64 [leaders + 1] or None, child_points int32 [rows * fanout] or None).
    ``global_ids`` / ``leader_ids`` int32 views of u32; ``leaders`` the
    leaders' own SQ8 payload (same padded_dim)."""
    if leaders.padded_dim != sq8.padded_dim:
        raise ValueError(f"leader padded_dim {leaders.padded_dim} != {sq8.padded_dim}")
    if global_ids.numel() != sq8.rows or leader_ids.numel() != leaders.rows:
        raise ValueError("one global id per row and per leader")
    dev = sq8.codes.device
    rows, nl = sq8.rows, leaders.rows
    child = torch.empty((rows, fanout_top), dtype=torch.int32, device=dev)
    point = torch.empty((rows, fanout_top), dtype=torch.int32, device=dev)
    offs = torch.empty(nl + 1, dtype=torch.int64, device=dev) if group else None
    pts = torch.empty(rows * fanout_top, dtype=torch.int32, device=dev) if group else None
    gi, li = global_ids.contiguous(), leader_ids.contiguous()
    N.check(N.load().tessa_global_d0_assign(
        _ptr(sq8.codes), _ptr(sq8.scales), _ptr(sq8.norms), _ptr(gi), rows, sq8.padded_dim, _ptr(leaders.codes),
        _ptr(leaders.scales), _ptr(leaders.norms), _ptr(li), nl, fanout_top, _ptr(child), _ptr(point),
        _ptr(offs) if group else None, _ptr(pts) if group else None, _stream_ptr(stream)), "global D0 assign")
    return child, point, offs, pts



@dataclass
class D0CapacityConfig:
    """d0_capacity.rs:22-47 defaults (params gpu_subtree_d0_capacity_*)."""

    enabled: bool = False
    high_ratio: float = 0.60
    target_ratio: float = 0.50
    low_ratio: float = 0.15
    min_efficient_rows: int = 32 * 1024
    quality_min_root_leaders: int = 64
    root_leader_cap: int = 10_000
    split_recursion_limit: int = 8


DEFAULT_GPU_WORKSPACE_BUDGET_BYTES = 512 * 1024 * 1024  # params.rs:2469
GPU_QUEUE_LEADER_STRIDE = 128


def find_max_admissible_rows(dim: int, leaf_knn: int, max_leaders_per_node: int, max_fanout: int,
                             workspace_budget_bytes: int | None, device_budget_bytes: int | None, c_max: int,
                             resident_format: int = N.RESIDENT_F32) -> int:
    return int(N.load().tessa_find_max_admissible_rows(dim, leaf_knn, max_leaders_per_node, max_fanout,
                                                       workspace_budget_bytes or 0, device_budget_bytes or 0, c_max,
                                                       resident_format))


def resident_admission(resident_rows: int, dim: int, leaf_knn: int, max_leaders_per_node: int, max_fanout: int,
                       workspace_budget_bytes: int | None, device_budget_bytes: int | None, c_max: int,
                       resident_format: int = N.RESIDENT_F32) -> N.ResidentAdmission:
    out = N.ResidentAdmission()
    N.check(N.load().tessa_plan_subtree_resident_admission(resident_rows, dim, leaf_knn, max_leaders_per_node,
                                                           max_fanout, workspace_budget_bytes or 0,
                                                           device_budget_bytes or 0, c_max, resident_format,
                                                           C.byref(out)), "resident admission")
    return out


def compute_thresholds(c_gpu: int, cfg: D0CapacityConfig = D0CapacityConfig()) -> N.D0Thresholds:
    return N.load().tessa_d0_compute_thresholds(c_gpu, cfg.high_ratio, cfg.target_ratio, cfg.low_ratio,
                                                cfg.min_efficient_rows)


def plan_root_leaders(total_points: int, root_fanout: int, t: N.D0Thresholds,
                      cfg: D0CapacityConfig = D0CapacityConfig()) -> dict:
    p = N.load().tessa_d0_plan_root_leaders(total_points, root_fanout, C.byref(t), cfg.quality_min_root_leaders,
                                            cfg.root_leader_cap)
    return {"k_capacity": p.k_capacity, "k_initial": p.k_initial, "root_leader_cap": p.root_leader_cap,
            "root_leader_source": N.D0_LEADER_SOURCES[p.source]}


def split_leader_count(rows: int, t: N.D0Thresholds) -> int:
    return int(N.load().tessa_d0_split_leader_count(rows, C.byref(t)))


def observe_child_unique_sizes(sizes, t: N.D0Thresholds) -> dict:
    a = np.ascontiguousarray(sizes, np.uint64)
    s = N.load().tessa_d0_observe_child_sizes(a.ctypes.data if len(a) else None, len(a), C.byref(t))
    return {f: getattr(s, f) for f, _ in N.D0ChildSummary._fields_}
