"""PGSQW1 SQ8 sidecar (shear_amd/sidecar.py): FNV-1a 64 against its
published test vectors, the header's byte positions, round trip and the
reader's checks (shear-core/src/algorithm/pipnn/dco_sq_int8.rs:476-527,
:1469-1475, :1595-1610, :2495-2651)."""
import struct

import numpy as np
import pytest

from shear_amd import sidecar as SC


def test_fnv1a64_published_vectors():
    assert SC.fnv1a64(b"") == 0xCBF29CE484222325
    assert SC.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert SC.fnv1a64(b"foobar") == 0x85944171F73967E8


def test_fingerprint_hashes_five_u64_fields():
    fp = SC.source_fingerprint(1000, 128, 8 + 1000 * 128 * 4)
    assert fp == SC.fnv1a64(b"".join(v.to_bytes(8, "little") for v in (1000, 128, 16, 8, 512008)))
    assert fp != SC.source_fingerprint(1000, 128, 8 + 1000 * 128 * 4, bits=4)


def test_round_trip_and_layout(tmp_path, orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 20)).astype(np.float32)
    codes, scales, norms = orc.quantize(x)
    h = SC.write_sidecar(tmp_path / "base", codes, scales, norms, 20)
    meta = (tmp_path / "base.meta").read_bytes()
    assert meta[:8] == b"PGSQW1\0\0" and struct.unpack_from("<II", meta, 8) == (1, 256)
    fields = struct.unpack_from("<13Q", meta, 16)
    assert fields[0:4] == (37, 20, codes.shape[1], 16) and fields[8:] == (37 * codes.shape[1], 37 * 8, 8, 0,
                                                                          codes.shape[1])
    assert meta[16 + 13 * 8:256] == bytes(256 - 16 - 13 * 8)
    assert len(meta) == 256 + 37 * 8 and (tmp_path / "base.codes").stat().st_size == codes.size
    assert struct.unpack_from("<2f", meta, 256) == (norms[0], scales[0])  # norm first, then scale
    h2, c2, s2, n2 = SC.read_sidecar(tmp_path / "base", rows=37, dim=20)
    assert h2 == h and np.array_equal(c2, codes) and np.array_equal(s2, scales) and np.array_equal(n2, norms)


def test_reader_checks(tmp_path, orc):
    codes, scales, norms = orc.quantize(np.ones((4, 8), np.float32))
    SC.write_sidecar(tmp_path / "s", codes, scales, norms, 8)
    with pytest.raises(SC.SidecarError, match="shape mismatch: sidecar rows=4 dim=8"):
        SC.read_sidecar(tmp_path / "s", rows=5, dim=8)
    with pytest.raises(SC.SidecarError, match="bits mismatch: sidecar=8 expected=4"):
        SC.read_sidecar(tmp_path / "s", rows=4, dim=8, bits=4)
    meta = bytearray((tmp_path / "s.meta").read_bytes())
    bad = bytes(meta)
    for off, val, msg in ((0, b"PGSQW2\0\0", "magic mismatch"), (8, struct.pack("<I", 2), "version 2"),
                          (12, struct.pack("<I", 128), "header size 128"),
                          (16 + 11 * 8, struct.pack("<Q", 7), "code layout 7")):
        m = bytearray(bad)
        m[off:off + len(val)] = val
        (tmp_path / "s.meta").write_bytes(bytes(m))
        with pytest.raises(SC.SidecarError, match=msg):
            SC.read_sidecar(tmp_path / "s")
