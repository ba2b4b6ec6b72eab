"""GPU-memory-aware task formation (libtessa_hip.so host code, no GPU work):
the reference's own d0_capacity tests (shear-core/src/algorithm/pipnn/
d0_capacity.rs:300-480) and the resident admission rule
(compute_backend.rs:1490-1522, estimates :898-930)."""
import pytest

from shear_amd import _native as N
from shear_amd import d0 as D


def thr(c_gpu, c_high, c_target, c_low):
    return N.D0Thresholds(c_gpu, c_high, c_target, c_low)


def test_default_config_ratios():  # d0_capacity.rs:305-310
    cfg = D.D0CapacityConfig()
    assert (cfg.high_ratio, cfg.target_ratio, cfg.low_ratio) == (0.60, 0.50, 0.15)


def test_thresholds_keep_order():  # :313-329
    t = D.compute_thresholds(1_000, D.D0CapacityConfig(high_ratio=0.85, target_ratio=0.75, low_ratio=0.20,
                                                       min_efficient_rows=32))
    assert (t.c_gpu, t.c_high, t.c_target, t.c_low) == (1_000, 850, 750, 200)


def test_thresholds_clamp_target():  # :331-344
    t = D.compute_thresholds(1_000, D.D0CapacityConfig(high_ratio=0.60, target_ratio=0.90, low_ratio=0.20,
                                                       min_efficient_rows=1))
    assert (t.c_high, t.c_target, t.c_low) == (600, 600, 200)
    assert (D.compute_thresholds(0).c_high, D.compute_thresholds(0).c_low) == (0, 0)


def test_root_leaders_capacity():  # :346-364
    p = D.plan_root_leaders(10_000_000, 6, thr(400_000, 340_000, 300_000, 64_000),
                            D.D0CapacityConfig(quality_min_root_leaders=64, root_leader_cap=10_000))
    assert p == {"k_capacity": 200, "k_initial": 200, "root_leader_cap": 10_000, "root_leader_source": "capacity"}


def test_root_leaders_quality_floor_and_cap():  # :366-394
    t = thr(1_000_000, 850_000, 750_000, 64_000)
    p = D.plan_root_leaders(1_000_000, 6, t, D.D0CapacityConfig(quality_min_root_leaders=128, root_leader_cap=10_000))
    assert (p["k_capacity"], p["k_initial"], p["root_leader_source"]) == (8, 128, "quality_floor")
    p = D.plan_root_leaders(20_000_000, 6, t, D.D0CapacityConfig(quality_min_root_leaders=160, root_leader_cap=100))
    assert (p["k_capacity"], p["k_initial"], p["root_leader_cap"], p["root_leader_source"]) == \
        (160, 100, 100, "root_leader_cap")


def test_resident_budget_tightens_admission():  # :396-446
    budget = 16 * 1024 ** 3
    args = (1024, 2, min(5000, D.GPU_QUEUE_LEADER_STRIDE), 3)
    workspace_only = D.find_max_admissible_rows(*args, budget, None, 1280)
    resident_aware = D.find_max_admissible_rows(*args, budget, budget, 1280)
    assert 0 < resident_aware < workspace_only
    cfg = D.D0CapacityConfig()
    p = D.plan_root_leaders(35_000_000, 6, D.compute_thresholds(resident_aware, cfg), cfg)
    assert p["k_capacity"] > cfg.quality_min_root_leaders
    assert p["k_initial"] == p["k_capacity"] and p["root_leader_source"] == "capacity"
    # the result is the admission boundary
    a = D.resident_admission(resident_aware, *args, budget, budget, 1280)
    b = D.resident_admission(resident_aware + 1, *args, budget, budget, 1280)
    assert a.plan.supported and not b.plan.supported
    assert b.plan.overflow_flags & (1 << 8) and b.device_admission_required_bytes > budget


def test_resident_estimates():
    a = D.resident_admission(1000, 100, 2, 128, 3, None, None, 1280)
    assert a.resident_device_bytes == 1000 * (100 * 4 + 4 + 4)  # f32 rows + id + norm
    assert a.device_admission_budget_bytes == 2 ** 64 - 1
    a = D.resident_admission(1000, 100, 2, 128, 3, None, None, 1280, N.RESIDENT_SQ8)
    assert a.resident_device_bytes == 1000 * (112 + 12)
    a = D.resident_admission(1000, 100, 2, 128, 3, None, None, 1280, N.RESIDENT_SQ4)
    assert a.resident_device_bytes == 1000 * (56 + 12)
    assert a.device_admission_required_bytes == a.resident_device_bytes + a.plan.required_bytes
    assert D.find_max_admissible_rows(0, 2, 128, 3, None, None, 1280) == 0


def test_split_leader_count():  # :448-458
    t = thr(400_000, 340_000, 300_000, 64_000)
    assert [D.split_leader_count(r, t) for r in (300_000, 341_000, 900_001)] == [1, 2, 4]


def test_child_size_observation():  # :460-479
    s = D.observe_child_unique_sizes([10, 100, 200, 300, 400_000], thr(400_000, 340_000, 300_000, 64))
    assert (s["max_rows"], s["p50_rows"], s["p95_rows"], s["p99_rows"]) == (400_000, 200, 400_000, 400_000)
    assert (s["oversized_count"], s["small_count"], s["small_rows"]) == (1, 1, 10)
