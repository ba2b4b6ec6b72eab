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
