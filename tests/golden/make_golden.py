"""Writes tests/golden/formula_fixtures.npz.

Inputs are the formula-generated data of the reference's own device tests
(paths relative to shear-core/src/algorithm/pipnn/):
  A  tessa_replay.rs:1800-1812  607 x 1024, ((r*17 + a*13) % 97) * 0.03125 - 1,
     row 7 copies row 6; one leaf of all rows; assignment over 16 leaders, r_h 2.
  B  tessa_replay.rs:1904-1913  leaves of 740, 728, 641 rows x 1024,
     ((r*131 + a*17 + r*a*3) % 251) * 0.0078125 - 0.75; assignment 64 x 16, r_h 2.
  C  compute_backend.rs:41972-41995  20 x 1024 codes ((r*13 + a*7) % 31) - 15,
     row 0 zero, rows 2/5 copy rows 1/4, scale 0.0078125*(1 + r%5),
     norm scale*scale*sum(code^2), global id 1000 - 7r, k 4.
The reference records no expected outputs for these (its tests only compare
its two GPU executors), so the expected outputs here come from the oracle;
every one is re-derived by the independent brute force in tests/brute.py
before the file is written.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

from oracle import pyoracle as orc  # noqa: E402
import brute  # noqa: E402

OUT = HERE / "formula_fixtures.npz"


def inputs_a():
    r = np.arange(607)[:, None]
    r = np.where(r == 7, 6, r)
    a = np.arange(1024)[None, :]
    return (((r * 17 + a * 13) % 97).astype(np.float32) * np.float32(0.03125) - np.float32(1.0)).astype(np.float32)


def inputs_b():
    rows = 740 + 728 + 641
    r = np.arange(rows, dtype=np.int64)[:, None]
    a = np.arange(1024, dtype=np.int64)[None, :]
    return (((r * 131 + a * 17 + r * a * 3) % 251).astype(np.float32) * np.float32(0.0078125)
            - np.float32(0.75)).astype(np.float32)


def inputs_c():
    r = np.arange(20)
    src = np.where(r == 2, 1, np.where(r == 5, 4, r))
    a = np.arange(1024)
    codes = (((src[:, None] * 13 + a[None, :] * 7) % 31) - 15).astype(np.int8)
    codes[src == 0] = 0
    scales = (np.float32(0.0078125) * (1 + (src % 5)).astype(np.float32)).astype(np.float32)
    sq = (codes.astype(np.int64) ** 2).sum(axis=1)
    norms = (scales * scales * sq.astype(np.float32)).astype(np.float32)
    gids = (1000 - 7 * r).astype(np.uint32)
    return codes, scales, norms, gids


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def leaf_case(codes, scales, norms, gids, sizes, k):
    members = np.arange(sum(sizes), dtype=np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint64)
    ids, d = orc.leaf_topk(codes, scales, norms, gids, members, offs, sizes, k)
    o = 0
    for off, n in zip(offs.tolist(), sizes):
        bid, bd = brute.leaf_topk(codes, scales, norms, gids, members[off:off + n], k)
        assert np.array_equal(ids[o:o + n * k], bid), "oracle and brute force disagree (ids)"
        assert np.array_equal(d[o:o + n * k].view(np.uint32), bd.view(np.uint32)), "distance bits"
        o += n * k
    return ids, d.view(np.uint32)


def assign_case(codes, scales, norms, gids, rows, leaders, r_h):
    members = np.arange(rows, dtype=np.uint32)
    lead = np.arange(leaders, dtype=np.uint32)
    ids, d = orc.assign_replay(codes, scales, norms, gids, members, lead, [0], [rows], [0], [leaders], [r_h])
    # brute force: 4-slot insertion with the tie key, leaders in slot order
    for m in range(rows):
        slots = []  # (d, leader)
        for l in lead.tolist():
            dd = brute.assign_dist(int(np.dot(codes[m].astype(np.int64), codes[l].astype(np.int64))), scales[m],
                                   norms[m], scales[l], norms[l])

            def before(x, y):
                if abs(np.float32(x[0] - y[0])) <= np.float32(2e-5):
                    kx = brute.hash64((m << 32) ^ x[1] ^ 0x9E3779B97F4A7C15)
                    ky = brute.hash64((m << 32) ^ y[1] ^ 0x9E3779B97F4A7C15)
                    return kx < ky or (kx == ky and x[1] < y[1])
                return x[0] < y[0]

            c = (dd, l)
            if len(slots) == 4 and not before(c, slots[-1]):
                continue
            slots.append(c)
            pos = len(slots) - 1
            while pos > 0 and before(c, slots[pos - 1]):
                slots[pos] = slots[pos - 1]
                pos -= 1
            slots[pos] = c
            slots = slots[:4]
        for q in range(r_h):
            assert ids[m * r_h + q] == gids[slots[q][1]], "assignment ids"
            assert d[m * r_h + q].view(np.uint32) == np.float32(slots[q][0]).view(np.uint32), "assignment dists"
    return ids, d.view(np.uint32)


def build():
    out = {}
    xa = inputs_a()
    ca, sa, na = orc.quantize(xa)
    ga = np.arange(607, dtype=np.uint32)
    out["a_digest"] = np.array(digest(ca, sa, na))
    for k in (2, 32):
        out[f"a_leaf_k{k}_ids"], out[f"a_leaf_k{k}_dbits"] = leaf_case(ca, sa, na, ga, [607], k)
    out["a_assign_ids"], out["a_assign_dbits"] = assign_case(ca, sa, na, ga, 607, 16, 2)

    xb = inputs_b()
    cb, sb, nb = orc.quantize(xb)
    gb = np.arange(xb.shape[0], dtype=np.uint32)
    out["b_digest"] = np.array(digest(cb, sb, nb))
    for k in (2, 32):
        out[f"b_leaf_k{k}_ids"], out[f"b_leaf_k{k}_dbits"] = leaf_case(cb, sb, nb, gb, [740, 728, 641], k)
    out["b_assign_ids"], out["b_assign_dbits"] = assign_case(cb, sb, nb, gb, 64, 16, 2)

    cc, sc, nc, gc = inputs_c()
    out["c_digest"] = np.array(digest(cc, sc, nc, gc))
    out["c_leaf_k4_ids"], out["c_leaf_k4_dbits"] = leaf_case(cc, sc, nc, gc, [20], 4)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    build()
