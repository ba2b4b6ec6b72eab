"""The PGSQW1 SQ8 sidecar: an SQ8 matrix on disk next to its .fbin source.

Host mirror of the reference's sidecar format (paths relative to
shear-core/src/algorithm/pipnn/dco_sq_int8.rs):

* ``<prefix>.codes``  the code rows, ``code_row_bytes`` each (dense i8 rows of
  padded_dim, or packed s4 at half of it), from offset 0 (:1469-1471, :670-677)
* ``<prefix>.meta``   a 256-byte header, then per row (norm f32, scale f32)
  little-endian (:1473-1475, :1595-1610, :680-694)
* header (:2495-2517): b"PGSQW1\\0\\0", version u32 1, header bytes u32 256,
  then u64 rows, dim, padded_dim, k_align, source_fbin_bytes, source_rows,
  source_dim, source_fingerprint, codes_bytes, meta_rows_bytes, bits,
  code layout (0 dense-i8, 1 packed-s4), code_row_bytes; zero padding
* fingerprint (:2632-2651): FNV-1a 64 over the little-endian bytes of rows,
  dim, k_align (16), bits, source_fbin_bytes
* checks on read (:476-527, :2520-2582) with the reference's messages.

The matrix itself comes from ``tessa.quantize_sq_int8_matrix`` on the GPU.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

MAGIC = b"PGSQW1\0\0"
VERSION = 1
HEADER_BYTES = 256
META_ROW_BYTES = 8
K_ALIGN = 16
LAYOUT_DENSE_I8, LAYOUT_PACKED_S4 = 0, 1
_FIELDS = ("rows", "dim", "padded_dim", "k_align", "source_fbin_bytes", "source_rows", "source_dim",
           "source_fingerprint", "codes_bytes", "meta_rows_bytes", "bits", "code_layout", "code_row_bytes")
_FNV_OFFSET = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3


class SidecarError(ValueError):
    pass


def fnv1a64(data: bytes, h: int = _FNV_OFFSET) -> int:
    for b in data:
        h = ((h ^ b) * _FNV_PRIME) & 0xFFFFFFFFFFFFFFFF
    return h


def source_fingerprint(rows: int, dim: int, source_fbin_bytes: int, bits: int = 8) -> int:
    return fnv1a64(struct.pack("<5Q", rows, dim, K_ALIGN, bits, source_fbin_bytes))


def code_row_bytes(padded_dim: int, layout: int) -> int:
    if layout == LAYOUT_DENSE_I8:
        return padded_dim
    if layout == LAYOUT_PACKED_S4:
        if padded_dim % 2:
            raise SidecarError(f"SQ+WMMA packed-s4 layout requires even padded_dim, got {padded_dim}")
        return padded_dim // 2
    raise SidecarError(f"Unsupported SQ+WMMA sidecar code layout {layout}")


def encode_header(h: dict) -> bytes:
    out = MAGIC + struct.pack("<II", VERSION, HEADER_BYTES) + struct.pack("<13Q", *(int(h[f]) for f in _FIELDS))
    return out + bytes(HEADER_BYTES - len(out))


def decode_header(buf: bytes) -> dict:
    if len(buf) < HEADER_BYTES:
        raise SidecarError("Failed to read SQ+WMMA sidecar header: short file")
    if buf[:8] != MAGIC:
        raise SidecarError("SQ+WMMA sidecar magic mismatch")
    version, hb = struct.unpack_from("<II", buf, 8)
    if version != VERSION:
        raise SidecarError(f"Unsupported SQ+WMMA sidecar version {version}")
    if hb != HEADER_BYTES:
        raise SidecarError(f"Unsupported SQ+WMMA sidecar header size {hb}")
    h = dict(zip(_FIELDS, struct.unpack_from("<13Q", buf, 16)))
    if h["bits"] == 0:
        h["bits"] = 8
    code_row_bytes(h["padded_dim"], h["code_layout"])  # layout check
    if h["code_row_bytes"] == 0:
        h["code_row_bytes"] = code_row_bytes(h["padded_dim"], h["code_layout"])
    return h


def validate(h: dict, rows: int, dim: int, bits: int = 8) -> None:
    """validate_for_dataset_with_bits (dco_sq_int8.rs:476-527)."""
    if not 4 <= bits <= 8:
        raise SidecarError(f"SQ-int8 bits must be in 4..=8, got {bits}")
    if h["rows"] != rows or h["dim"] != dim or h["source_rows"] != rows or h["source_dim"] != dim:
        raise SidecarError(f"SQ+WMMA sidecar shape mismatch: sidecar rows={h['rows']} dim={h['dim']} "
                           f"source_rows={h['source_rows']} source_dim={h['source_dim']} expected rows={rows} dim={dim}")
    if h["k_align"] != K_ALIGN:
        raise SidecarError(f"SQ+WMMA sidecar k_align mismatch: sidecar={h['k_align']} expected={K_ALIGN}")
    if h["bits"] != bits:
        raise SidecarError(f"SQ+WMMA sidecar bits mismatch: sidecar={h['bits']} expected={bits}")
    want = code_row_bytes(h["padded_dim"], h["code_layout"])
    if h["code_row_bytes"] != want:
        layout = "dense-i8" if h["code_layout"] == LAYOUT_DENSE_I8 else "packed-s4"
        raise SidecarError(f"SQ+WMMA sidecar code_row_bytes mismatch: sidecar={h['code_row_bytes']} "
                           f"expected={want} layout={layout}")
    if h["codes_bytes"] != h["rows"] * h["code_row_bytes"]:
        raise SidecarError(f"SQ+WMMA sidecar codes_bytes mismatch: sidecar={h['codes_bytes']} "
                           f"expected={h['rows'] * h['code_row_bytes']} rows={h['rows']} "
                           f"code_row_bytes={h['code_row_bytes']}")


def write_sidecar(prefix, codes: np.ndarray, scales: np.ndarray, norms: np.ndarray, dim: int,
                  source_fbin_bytes: int | None = None, bits: int = 8) -> dict:
    """Write ``<prefix>.codes`` and ``<prefix>.meta`` for a dense-i8 SQ8 matrix
    (host arrays, e.g. an Sq8Matrix's tensors after ``.cpu()``).  The source
    .fbin size defaults to 8 + rows * dim * 4."""
    codes = np.ascontiguousarray(codes, np.int8)
    rows, pd = codes.shape
    fbin = 8 + rows * dim * 4 if source_fbin_bytes is None else int(source_fbin_bytes)
    h = {"rows": rows, "dim": dim, "padded_dim": pd, "k_align": K_ALIGN, "source_fbin_bytes": fbin,
         "source_rows": rows, "source_dim": dim, "source_fingerprint": source_fingerprint(rows, dim, fbin, bits),
         "codes_bytes": rows * pd, "meta_rows_bytes": rows * META_ROW_BYTES, "bits": bits,
         "code_layout": LAYOUT_DENSE_I8, "code_row_bytes": pd}
    meta = np.empty((rows, 2), "<f4")
    meta[:, 0] = np.asarray(norms, np.float32)
    meta[:, 1] = np.asarray(scales, np.float32)
    Path(f"{prefix}.codes").write_bytes(codes.tobytes())
    Path(f"{prefix}.meta").write_bytes(encode_header(h) + meta.tobytes())
    return h


def read_sidecar(prefix, rows: int | None = None, dim: int | None = None, bits: int = 8):
    """(header, codes int8 [rows, code_row_bytes], scales f32, norms f32),
    checked against (rows, dim) when given."""
    meta = Path(f"{prefix}.meta").read_bytes()
    h = decode_header(meta[:HEADER_BYTES])
    if rows is not None or dim is not None:
        validate(h, h["rows"] if rows is None else rows, h["dim"] if dim is None else dim, bits)
    m = np.frombuffer(meta, "<f4", count=2 * h["rows"], offset=HEADER_BYTES).reshape(-1, 2)
    codes = np.fromfile(f"{prefix}.codes", np.int8, count=h["codes_bytes"]).reshape(h["rows"], h["code_row_bytes"])
    return h, codes, m[:, 1].copy(), m[:, 0].copy()
