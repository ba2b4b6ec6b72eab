"""TierLift spill artifacts (shear_amd/spill.py): the reference's part-file
names, record bytes, segment manifest and rollover
(shear-core/src/algorithm/pipnn/spill_hashprune.rs:139-145, :231-238,
:727-851), read back with checks; the HashPrune result over the read-back
records equals the one over the original stream (the reservoirs do not
depend on record order)."""
import struct

import numpy as np
import pytest

from shear_amd import spill as SP
from test_hashprune_oracle import random_stream


def test_names_bytes_and_manifest(tmp_path):
    r = np.zeros(3, SP.EDGE_RECORD_DTYPE)
    r["src"] = [5, 1_000_002, 2]
    r["dst"] = [7, 8, 9]
    r["hash"] = [0x1234, 1, 2]
    r["flags"] = [0, 0, 3]
    r["dist"] = [0.5, 1.5, 2.5]
    parts, segs, manifest = SP.write_spill_artifacts(tmp_path / "cand.bin", r)
    assert [p.name for p in parts] == ["cand_shard00000_part000.log", "cand_shard00001_part000.log"]
    assert manifest.name == "candidate_segments.manifest"
    assert manifest.read_text() == "0,0,0,32,2,2,5,1\n1,0,0,16,1,1000002,1000002,1\n"
    raw = parts[0].read_bytes()
    assert raw[:16] == struct.pack("<IIHHf", 2, 9, 2, 3, 2.5)  # sorted by src inside the segment
    assert raw[16:] == struct.pack("<IIHHf", 5, 7, 0x1234, 0, 0.5)


def test_segments_rollover_and_round_trip(tmp_path, orc):
    rng = np.random.default_rng(3)
    r = random_stream(rng, 3000, 50000, 12, 500)
    parts, segs, _ = SP.write_spill_artifacts(tmp_path / "c", r, shard_points=1000, segment_records=4000,
                                              part_max_bytes=16 * 9000)
    assert len({s.shard_id for s in segs}) == 3
    assert any(s.file_id > 0 for s in segs)  # parts rolled over
    assert all(s.record_count <= 4000 and s.byte_offset + s.byte_len <= 16 * 9000 for s in segs)
    back = SP.read_spill_artifacts(tmp_path / "c", shard_points=1000)
    key = lambda a: np.sort(a.view(np.uint8).reshape(-1, 16).view("V16").ravel())
    assert np.array_equal(key(back), key(r))
    want = orc.hashprune_reduce(3000, 64, r)
    got = orc.hashprune_reduce(3000, 64, back)
    assert all(np.array_equal(a, b) for a, b in zip(want, got))


def test_reader_checks(tmp_path):
    r = np.zeros(4, SP.EDGE_RECORD_DTYPE)
    r["src"] = [3, 1, 2, 0]
    parts, _, manifest = SP.write_spill_artifacts(tmp_path / "c", r)
    raw = bytearray(parts[0].read_bytes())
    raw[0:4], raw[16:20] = raw[16:20], raw[0:4]  # out of src order
    parts[0].write_bytes(bytes(raw))
    with pytest.raises(SP.SpillError, match="not sorted by src"):
        SP.read_spill_artifacts(tmp_path / "c")
    manifest.write_text("0,0,0,64,4,0,3\n")
    with pytest.raises(SP.SpillError, match="expected 8 fields"):
        SP.read_spill_artifacts(tmp_path / "c")
