"""Independent brute-force restatements used to pin the oracle on small inputs.

Written from the reference text without sharing code with oracle/: float32
arithmetic goes through numpy scalars one IEEE operation at a time, integer
dots through int64 numpy products, and the row insertion is plain Python.
"""
from __future__ import annotations

import numpy as np

EPS = np.float32(2.0e-5)
F32 = np.float32


def quantize_row(x: np.ndarray, max_code: float = 127.0):
    """dco_sq_int8.rs:1431-1467 with numpy float32 scalars."""
    max_abs = F32(0.0)
    norm = F32(0.0)
    for v in x.astype(np.float32):
        if not np.isfinite(v):
            raise ValueError("non-finite")
        max_abs = max(max_abs, F32(abs(v)))
        norm = F32(norm + F32(v * v))
    if max_abs == 0:
        return np.zeros(len(x), np.int8), F32(1.0), norm
    mc = F32(max_code)
    scale = F32(max_abs / mc)
    codes = []
    for v in x.astype(np.float32):
        q = F32(v / scale)
        # half away from zero; float(q) + 0.5 is exact in float64
        r = float(np.floor(abs(float(q)) + 0.5)) * (1.0 if q >= 0 else -1.0)
        codes.append(int(min(max(r, -mc), mc)))
    return np.array(codes, np.int8), scale, norm


def leaf_dist(dot: int, rs, rn, cs, cn) -> np.float32:
    """(rn + cn) + (-2 * ((rs * cs) * f32(dot))), one rounding per op."""
    sc = F32(F32(rs) * F32(cs))
    u = F32(sc * F32(dot))
    w = F32(F32(-2.0) * u)
    d = F32(F32(F32(rn) + F32(cn)) + w)
    return F32(0.0) if d <= 0 else d


def assign_dist(dot: int, ps, pn, ls, ln) -> np.float32:
    a = F32(F32(2.0) * F32(ps))
    b = F32(a * F32(ls))
    c = F32(b * F32(dot))
    d = F32(F32(F32(pn) + F32(ln)) - c)
    return F32(0.0) if d <= 0 else d


def beats(dc, idc, ds, ids) -> bool:
    delta = F32(F32(dc) - F32(ds))
    if abs(delta) <= EPS:
        return idc < ids
    return F32(dc) < F32(ds)


def rowtopk(k: int, stream):
    """leaf_build.rs:887-957 over an iterable of (dist, id)."""
    buf: list[tuple[np.float32, int]] = []
    for d, i in stream:
        if k == 0:
            continue
        if len(buf) < k:
            pos = len(buf)
            buf.append((d, i))
            while pos > 0 and beats(d, i, *buf[pos - 1]):
                buf[pos] = buf[pos - 1]
                pos -= 1
            buf[pos] = (d, i)
        else:
            if not beats(d, i, *buf[k - 1]):
                continue
            pos = k - 1
            while pos > 0 and beats(d, i, *buf[pos - 1]):
                buf[pos] = buf[pos - 1]
                pos -= 1
            buf[pos] = (d, i)
    return buf


def leaf_topk(codes, scales, norms, gids, members, k):
    """One leaf: every member row against every other member in member order."""
    members = np.asarray(members)
    c = codes[members].astype(np.int64)
    dots = c @ c.T
    n = len(members)
    keff = min(k, n - 1)
    out_ids = np.full((n, k), 0xFFFFFFFF, np.uint32)
    out_d = np.full((n, k), np.finfo(np.float32).max, np.float32)
    for r in range(n):
        mr = members[r]
        stream = ((leaf_dist(int(dots[r, j]), scales[mr], norms[mr], scales[members[j]], norms[members[j]]),
                   int(gids[members[j]])) for j in range(n) if j != r)
        buf = rowtopk(keff, stream)
        for q, (d, i) in enumerate(buf):
            out_ids[r, q] = i
            out_d[r, q] = d
    return out_ids.reshape(-1), out_d.reshape(-1)


def hash64(v: int) -> int:
    m = (1 << 64) - 1
    v ^= v >> 30
    v = (v * 0xBF58476D1CE4E5B9) & m
    v ^= v >> 27
    v = (v * 0x94D049BB133111EB) & m
    return v ^ (v >> 31)
