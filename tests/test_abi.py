"""The C ABI library loads and exports every symbol include/tessa_hip.h declares
(no compute calls: these run on a CPU-only machine)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from shear_amd import _native as N

HEADER = Path(__file__).resolve().parent.parent / "include" / "tessa_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tessa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("tessa_leaf_topk", "tessa_assign_replay", "tessa_sq8_quantize", "tessa_session_create",
                 "tessa_session_destroy", "tessa_session_upload_sq8", "tessa_session_leaf_topk",
                 "tessa_session_assign_replay", "tessa_query_caps", "tessa_overflow_labels", "tessa_abi_version"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = N.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(N.SIGNATURES), "ctypes signatures cover the header"


def test_abi_version_and_labels_without_gpu():
    lib = N.load()
    assert lib.tessa_abi_version() == 1
    assert N.overflow_labels(0) == "none"
    assert N.overflow_labels((1 << 0) | (1 << 3)) == "QUEUE_NODE|LEAF_ROW"
    assert N.overflow_labels(1 << 40) == "UNKNOWN_0x10000000000"
    assert N.overflow_labels((1 << 11) | (1 << 50)) == "WATCHDOG_STALLED|UNKNOWN_0x4000000000000"


def test_struct_layouts_match_header_sizes():
    # tessa_status: i32 + u32 + u64 + 512 chars
    assert C.sizeof(N.TessaStatus) == 8 + 8 + 512
    assert C.sizeof(N.LeafBatch) == 4 * 8 + 6 * 4
    assert C.sizeof(N.Sq8View) == 4 * 8 + 8 + 4 + 4
    assert C.sizeof(N.EdgeRecord) == 16  # SpillRecord16
    assert C.sizeof(N.SketchView) == 8 + 8 + 4 + 4


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        N.load(tmp_path / "absent.so")


def test_struct_layouts_match_the_c_compiler(tmp_path):
    # sizes and field offsets of the header's structs as gcc lays them out,
    # against the ctypes mirrors
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    specs = {
        "tessa_subtree_plan": (N.SubtreePlan, ["supported", "required_bytes", "budget_bytes"]),
        "tessa_resident_admission": (N.ResidentAdmission, ["plan", "resident_device_bytes",
                                                           "device_admission_budget_bytes"]),
        "tessa_d0_thresholds": (N.D0Thresholds, ["c_gpu", "c_low"]),
        "tessa_d0_leader_plan": (N.D0LeaderPlan, ["k_capacity", "source"]),
        "tessa_d0_child_summary": (N.D0ChildSummary, ["max_rows", "small_rows"]),
        "tessa_captured_assignment": (N.CapturedAssignment, ["depth", "leader_count", "member_offset",
                                                             "leader_offset"]),
        "tessa_hashprune_backfill": (N.HashPruneBackfill, ["mode", "hash_quota", "max_backfill_per_row",
                                                           "soft_tier_priority_alpha"]),
        "tessa_tierlift_config": (N.TierLiftConfig, ["spill_base", "l_max", "threads", "expected_records"]),
        "tessa_tierlift_stats": (N.TierLiftStats, ["shards", "threads", "route_s", "reduce_s", "unique_records"]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for name, (_, fields) in specs.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for name, (cls, fields) in specs.items():
        assert int(got[name]) == C.sizeof(cls), name
        for f in fields:
            assert int(got[f"{name}.{f}"]) == getattr(cls, f).offset, f"{name}.{f}"


@pytest.mark.parametrize("policy,l_max,code,text", [
    ((9, 0, 0, 0.0), 64, 4, "not a named R-half policy"),
    ((3, 0, 33, 0.0), 64, 1, "1..=floor(l_max/2), got cap=33 l_max=64"),
    ((1, 4, 0, 0.0), 64, 1, "hash quota must be in 1..=3"),
    ((3, 0, 0, 0.99), 64, 1, "finite and >= 1.0"),
    ((3, 0, 0, float("inf")), 64, 1, "finite and >= 1.0"),
    ((2, 0, 0, 1.05), 64, 1, "SoftTier priority alpha"),  # alpha is SoftTier's only
    ((3, 0, 1, 0.0), 1, 1, "got cap=1 l_max=1"),
])
def test_backfill_policy_validation_without_gpu(policy, l_max, code, text):
    # params.rs:2696-2729: the policy is checked before any device work
    # (codes: 1 TESSA_ERR_INVALID_ARGUMENT, 4 TESSA_ERR_UNSUPPORTED)
    lib = N.load()
    h = C.c_void_p()
    st = lib.tessa_hashprune_create_backfill(16, l_max, C.byref(N.HashPruneBackfill(*policy)), C.byref(h))
    assert st.code == code and not h.value
    assert text in st.msg.decode()
