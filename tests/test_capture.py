"""TESSA capture writer (shear_amd/capture.py): the reference's own capture
tests (shear-core/src/algorithm/pipnn/tessa_capture.rs:1137-1470) restated,
the hash building blocks against published vectors (FNV-1a 64, SplitMix64),
and finalize (tessa_replay.rs:240-318)."""
import hashlib
import json
import struct

import numpy as np
import pytest

from shear_amd import capture as CP


def assignment_task(i, rows, leaders):  # tessa_capture.rs:1137-1151
    return CP.make_assignment_task(42, 1, i, min(leaders, 8), 1024,
                                   [(i * 10_007 + r) % 1_000_000 for r in range(rows)][::-1],
                                   [(i * 257 + l) % 1_000_000 for l in range(leaders)])


def leaf_task(i, rows):  # :1153-1163
    return CP.make_leaf_task(42, 2, 1024, [(i * 4099 + r) % 1_000_000 for r in range(rows)][::-1])


def hex_digest(b):
    return f"{b:02x}" * 32


def dataset():
    return {"canonical_base_path": "/data/base.fbin", "rows": 1_000_000, "dimension": 128,
            "header_sha256": hex_digest(0x11)}


def provenance(seed=42):
    return {"seed": seed, "git_commit": "abc", "binary_sha256": hex_digest(0x22), "command_sha256": hex_digest(0x33),
            "root_leader_hash": 11, "d0_partition_hash": 13, "d0_task_list_hash": 17}


def small_selection():
    s = CP.TessaCaptureSampler(42)
    s.observe_assignment(assignment_task(1, 256, 16))
    s.observe_assignment(assignment_task(2, 513, 17))
    s.observe_leaf(leaf_task(3, 256))
    return s.finish()


def test_hash_building_blocks():
    f = CP._Fnv(b"")
    assert f.h == 0xCBF29CE484222325
    f.write(b"foobar")
    assert f.h == 0x85944171F73967E8
    assert CP.mix_membership_id(0) == 0xE220A8397B1DCDAF  # SplitMix64's first output from state 0
    # the digest is order independent; hashes depend on every field
    assert CP.membership_digest([5, 9, 1]) == CP.membership_digest([1, 5, 9])
    a = CP.make_leaf_task(42, 2, 1024, [3, 1, 2])
    assert a.member_ids == [1, 2, 3] and a.priority == CP.priority_for_task(42, a.task_hash)
    assert a.task_hash != CP.make_leaf_task(43, 2, 1024, [1, 2, 3]).task_hash
    assert a.task_hash != CP.make_leaf_task(42, 3, 1024, [1, 2, 3]).task_hash


def test_bin_boundaries_are_exact():  # :1165-1190
    assert [CP.assignment_row_bin(r) for r in (255, 256, 1024, 1025, 8192, 8193)] == [None, 0, 0, 1, 1, 2]
    assert [CP.assignment_leader_bin(l) for l in (0, 16, 17, 32, 33, 64, 65, 128, 129)] == \
        [None, 0, 1, 1, 2, 2, 3, 3, None]
    assert [CP.leaf_size_bin(r) for r in (255, 256, 512, 513, 896, 897, 1280, 1281)] == \
        [None, 0, 0, 1, 1, 2, 2, None]


def test_dataset_metadata_hashes_the_fbin_header(tmp_path):  # :1192-1216
    p = tmp_path / "base.fbin"
    p.write_bytes(struct.pack("<ii", 3, 2) + bytes(24))
    m = CP.dataset_metadata(p)
    assert (m["rows"], m["dimension"], m["canonical_base_path"]) == (3, 2, str(p.resolve()))
    assert m["header_sha256"] == hashlib.sha256(struct.pack("<ii", 3, 2)).hexdigest()


def test_bottom_k_is_order_independent_and_bounded():  # :1217-1304
    assignments, leaves, i = [], [], 0
    for rows in (256, 1025, 8193):
        for leaders in (16, 17, 33, 65):
            for _ in range(20):
                assignments.append(assignment_task(i, rows, leaders))
                i += 1
    for rows in (256, 513, 897):
        for _ in range(70):
            leaves.append(leaf_task(i, rows))
            i += 1

    def select(ao, lo):
        s = CP.TessaCaptureSampler(42)
        for j in ao:
            s.observe_assignment(assignments[j])
        for j in lo:
            s.observe_leaf(leaves[j])
        return s.finish()

    fwd = select(range(len(assignments)), range(len(leaves)))
    rev = select(reversed(range(len(assignments))), reversed(range(len(leaves))))
    shf = select(sorted(range(len(assignments)), key=lambda j: assignments[j].priority ^ 0xA5A5A5A5),
                 sorted(range(len(leaves)), key=lambda j: leaves[j].priority ^ 0x5A5A5A5A))
    for other in (rev, shf):
        assert [t.task_hash for t in fwd.assignment_tasks] == [t.task_hash for t in other.assignment_tasks]
        assert [t.task_hash for t in fwd.leaf_tasks] == [t.task_hash for t in other.leaf_tasks]
    assert len(fwd.assignment_tasks) == 12 * 16 and len(fwd.leaf_tasks) == 3 * 64
    assert fwd.bin_counts.assignment_observed == [[20] * 4] * 3
    assert fwd.bin_counts.assignment_selected == [[16] * 4] * 3
    assert fwd.bin_counts.leaf_observed == [70] * 3 and fwd.bin_counts.leaf_selected == [64] * 3


def test_fragment_round_trip_merge_and_idempotency(tmp_path):  # :1306-1351
    first = small_selection()
    p = CP.write_tessa_capture_fragment(tmp_path, 0x11, first)
    b = p.read_bytes()
    assert p.name == "fragment-0000000000000011.json" and b.endswith(b"}\n")
    assert CP.write_tessa_capture_fragment(tmp_path, 0x11, first) == p and p.read_bytes() == b
    conflicting = small_selection()
    conflicting.bin_counts.leaf_observed[0] += 1
    with pytest.raises(CP.CaptureError, match="differs from request 0000000000000011"):
        CP.write_tessa_capture_fragment(tmp_path, 0x11, conflicting)
    s2 = CP.TessaCaptureSampler(42)
    s2.observe_leaf(leaf_task(4, 513))
    CP.write_tessa_capture_fragment(tmp_path, 0x22, s2.finish())
    merged = CP.merge_tessa_capture_fragments(tmp_path, 42)
    assert len(merged.assignment_tasks) == 2 and len(merged.leaf_tasks) == 2
    assert merged.bin_counts.leaf_observed == [1, 1, 0]


def test_capture_write_load_and_rejections(tmp_path):  # :1353-1470
    path = CP.write_tessa_capture(tmp_path / "ok", dataset(), provenance(), small_selection())
    m = json.loads(path.read_bytes())
    assert list(m) == ["version", "dataset", "provenance", "bin_counts", "files", "assignment_tasks", "leaf_tasks"]
    _, sel = CP.load_tessa_capture(tmp_path / "ok", dataset())
    assert [t.task_hash for t in sel.leaf_tasks] == [t.task_hash for t in small_selection().leaf_tasks]
    assert (tmp_path / "ok" / CP.ASSIGNMENT_MEMBERS_FILE).stat().st_size == 4 * (256 + 513)
    with pytest.raises(CP.CaptureError, match="identity mismatch"):
        CP.load_tessa_capture(tmp_path / "ok", dict(dataset(), header_sha256=hex_digest(0xFF)))
    # duplicate task hash
    CP.write_tessa_capture(tmp_path / "dup", dataset(), provenance(), small_selection())
    mm = json.loads((tmp_path / "dup" / CP.MANIFEST_FILE).read_bytes())
    mm["assignment_tasks"][1]["task_hash"] = mm["assignment_tasks"][0]["task_hash"]
    (tmp_path / "dup" / CP.MANIFEST_FILE).write_text(json.dumps(mm))
    with pytest.raises(CP.CaptureError):
        CP.load_tessa_capture(tmp_path / "dup")
    # a member id outside the dataset
    CP.write_tessa_capture(tmp_path / "oor", dataset(), provenance(), small_selection())
    f = tmp_path / "oor" / CP.ASSIGNMENT_MEMBERS_FILE
    b = bytearray(f.read_bytes())
    b[:4] = struct.pack("<I", dataset()["rows"])
    f.write_bytes(bytes(b))
    with pytest.raises(CP.CaptureError):
        CP.load_tessa_capture(tmp_path / "oor")
    with pytest.raises(CP.CaptureError, match="invalid TESSA capture provenance"):
        CP.write_tessa_capture(tmp_path / "bad", dataset(), dict(provenance(), root_leader_hash=0), small_selection())


def test_finalize(tmp_path):
    CP.write_tessa_capture_fragment(tmp_path / "frag", 0x1, small_selection())
    (tmp_path / "prov.json").write_text(json.dumps({"dataset": dataset(), "provenance": provenance()}))
    prof = {"root_fanout": {"root_leader_hash": 11}, "gpu_subtree": {"d0_partition_hash": 13, "d0_task_list_hash": 17}}
    (tmp_path / "profile.json").write_text(json.dumps(prof))
    out = CP.finalize_tessa_capture(tmp_path / "frag", tmp_path / "profile.json", tmp_path / "prov.json",
                                    tmp_path / "out", 42)
    assert out.name == "manifest.json" and len(CP.load_tessa_capture(tmp_path / "out")[1].leaf_tasks) == 1
    with pytest.raises(CP.CaptureError, match="capture seed mismatch: requested=7 provenance=42"):
        CP.finalize_tessa_capture(tmp_path / "frag", tmp_path / "profile.json", tmp_path / "prov.json",
                                  tmp_path / "out2", 7)
    prof["gpu_subtree"]["d0_task_list_hash"] = 18
    (tmp_path / "profile.json").write_text(json.dumps(prof))
    with pytest.raises(CP.CaptureError, match="d0_task_list_hash mismatch: profile=18 provenance=17"):
        CP.finalize_tessa_capture(tmp_path / "frag", tmp_path / "profile.json", tmp_path / "prov.json",
                                  tmp_path / "out3", 42)
