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


# ---- subtree partition ---------------------------------------------------------

M64 = (1 << 64) - 1


def tie_key(point: int, leader: int) -> int:
    return hash64(((point << 32) ^ leader ^ 0x9E3779B97F4A7C15) & M64)


def assign_before(d, p, l, od, ol) -> bool:
    """compute_backend.rs:6541-6568."""
    if abs(F32(F32(d) - F32(od))) <= EPS:
        a, b = tie_key(p, l), tie_key(p, ol)
        return a < b or (a == b and l < ol)
    return F32(d) < F32(od)


def adaptive_psamp(base, n: int, depth: int) -> np.float32:
    f = F32(base)
    for lim, m in ((20_000_000, 0.05), (10_000_000, 0.1), (5_000_000, 0.2), (1_000_000, 0.4), (100_000, 0.7)):
        if n >= lim:
            f = F32(f * F32(m))
            break
    if depth > 4:
        f = F32(f * F32(0.35))
    elif depth > 2:
        f = F32(f * F32(0.5))
    elif depth > 0:
        f = F32(f * F32(0.8))
    return min(max(f, F32(0.00005)), F32(0.1))


def meaningful(parent: int, max_child: int, terminal: int) -> bool:
    if parent <= terminal or max_child <= terminal:
        return True
    if max_child >= parent:
        return False
    shrink = max(parent >> 5, 32)
    if shrink >= parent:
        shrink = 1
    return max_child + shrink <= parent


def partition(codes, scales, norms, *, seed, root_depth=0, max_depth=10, max_leaders=128, fanout_second=1,
              leaf_min=64, leaf_max=256, small_node_limit=4096, psamp=0.001, root_leaders=None):
    """Level-order RBC split (compute_backend.rs:12456-13078, 15047-15727):
    -> (leaves as lists of row ids, flags).  Children keep the parent's row
    order; nodes of a level are processed in publication order."""
    R = len(codes)
    c64 = codes.astype(np.int64)
    roots = [] if root_leaders is None else [int(x) for x in root_leaders]

    def best(p, leaders, F):
        bd = [F32(np.finfo(np.float32).max)] * F
        bs = [None] * F
        bl = [0xFFFFFFFF] * F
        dots = c64[leaders] @ c64[p]
        for s, l in enumerate(leaders):
            d = assign_dist(int(dots[s]), scales[p], norms[p], scales[l], norms[l])
            if not assign_before(d, p, l, bd[F - 1], bl[F - 1]):
                continue
            pos = F - 1
            while pos > 0 and assign_before(d, p, l, bd[pos - 1], bl[pos - 1]):
                bd[pos], bs[pos], bl[pos] = bd[pos - 1], bs[pos - 1], bl[pos - 1]
                pos -= 1
            bd[pos], bs[pos], bl[pos] = d, s, l
        return bs

    def base_count(n, depth, cap):
        b = int(F32(F32(adaptive_psamp(psamp, n, depth) * F32(n)) + F32(0.5)))
        return min(max(b, 2), cap)

    leaves, flags = [], 0
    level = [(list(range(R)), root_depth, seed & M64)] if R else []
    while level and not flags:
        nxt = []
        for rows, depth, nseed in level:
            n = len(rows)
            rel = max(depth - root_depth, 0)
            probe = rel == 0 and fanout_second > 1 and n > 1
            if n > leaf_max or (probe and n * fanout_second > small_node_limit):
                # ---- large node
                if depth >= max_depth:
                    flags |= 1 << 10
                    continue
                max_l = max(2, min(max_leaders, min(max(n, 2), 128)))
                use_root = rel == 0 and len(roots) > 0
                L = min(len(roots) if use_root else base_count(n, depth, max_l), max_l)
                F = min(max(fanout_second if rel == 0 else 1, 1), L)
                leaders = roots[:L] if use_root else [rows[min(s * n // L, n - 1)] for s in range(L)]
                attempt = 0
                while True:
                    slots = [best(p, leaders, F) for p in rows]
                    counts = [0] * L
                    for sl in slots:
                        for s in sl:
                            counts[s] += 1
                    nonempty = sum(1 for c in counts if c)
                    if nonempty > 1 and meaningful(n, max(counts), leaf_max):
                        children = [[p for p, sl in zip(rows, slots) if s in sl] for s in range(L)]
                        break
                    if not use_root and (attempt == 0 or L < max_l):
                        nl = L if attempt == 0 else (2 * L if 2 * L < max_l else max_l)
                        attempt += 1
                        new = []
                        for s in range(nl):
                            b, e = s * n // nl, (s + 1) * n // nl
                            e = max(e, b + 1)
                            key = hash64((nseed ^ ((attempt * 0xD6E8FEB86659FD93) & M64)
                                          ^ ((s * 0x9E3779B97F4A7C15) & M64)) & M64)
                            new.append(rows[b + key % (e - b)])
                        leaders, L = new, nl
                        continue
                    children = [rows[0::2], rows[1::2]]
                    break
                for s, ch in enumerate(children):
                    if not ch:
                        continue
                    if len(ch) <= leaf_max:
                        leaves.append(ch)
                    elif depth + 1 >= max_depth:
                        flags |= 1 << 10
                        break
                    else:
                        cs = nseed ^ ((s * 0x94D049BB133111EB) & M64) ^ ((len(ch) << 23) & M64)
                        nxt.append((ch, depth + 1, cs))
            else:
                # ---- small node (process_node)
                pts = sorted(set(rows))
                n = len(pts)
                if n <= leaf_max and not probe:
                    leaves.append(pts)
                    continue
                if depth >= max_depth:
                    flags |= 1 << 10
                    continue
                max_l = max(min(max_leaders, n), 2)
                if max_l > 128:
                    flags |= 1 << 4
                    continue
                base = base_count(n, depth, max_l)
                use_root = rel == 0 and len(roots) > 0
                ok, kids = False, []
                for attempt in range(1 if use_root else 6):
                    L = min(len(roots) if use_root else base << attempt, max_l)
                    if use_root:
                        leaders = roots[:L]
                    else:
                        keyed = sorted((hash64((nseed ^ ((attempt * 0xBF58476D1CE4E5B9) & M64) ^ (depth << 19)
                                                ^ (i << 7) ^ ((p << 31) & M64)) & M64), p)
                                       for i, p in enumerate(pts))
                        leaders = [p for _, p in keyed[:L]]
                    F = min(max(fanout_second if rel == 0 else 1, 1), L)
                    slots = [best(p, leaders, F) for p in pts]
                    kids, small, maxc = [], [], 0
                    for s in range(L):
                        ch = sorted({p for p, sl in zip(pts, slots) if s in sl})
                        if not ch:
                            continue
                        if len(ch) < leaf_min:
                            small = sorted(set(small) | set(ch))
                            if len(small) >= leaf_min:
                                kids.append(small)
                                maxc = max(maxc, len(small))
                                small = []
                        else:
                            kids.append(ch)
                            maxc = max(maxc, len(ch))
                    if small:
                        if kids and len(kids[-1]) + len(small) <= leaf_max:
                            kids[-1] = sorted(set(kids[-1]) | set(small))
                            maxc = max(maxc, len(kids[-1]))
                        else:
                            kids.append(small)
                            maxc = max(maxc, len(small))
                    if len(kids) > 1 and meaningful(n, maxc, leaf_max):
                        ok = True
                        break
                    if L >= max_l:
                        break
                if not ok:
                    leaves.append(pts)
                else:
                    leaves.extend(kids)
        level = nxt
    return leaves, flags


# ---- candidate records -> edges (leaf_build.rs:1679-1829) ---------------------------

def compute_hash(sp, sc, m_bits: int) -> int:
    """hash_prune.rs:2239-2251, vectorised over the bits."""
    diff = np.asarray(sc, np.float32)[:m_bits] - np.asarray(sp, np.float32)[:m_bits]
    bits = (diff >= np.float32(0)).astype(np.uint32)
    return int((bits << np.arange(m_bits, dtype=np.uint32)).sum())


def flush_edges(point_ids, k, topk_ids, topk_dists, sketches, m_bits):
    """List of (src, dst, hash, flags, dist bits) in the reference's push order."""
    pids = np.asarray(point_ids, np.uint32)
    members = set(int(p) for p in pids)
    ids = np.asarray(topk_ids, np.uint32).reshape(len(pids), k) if k else np.zeros((len(pids), 0), np.uint32)
    ds = np.asarray(topk_dists, np.float32).reshape(len(pids), k) if k else np.zeros((len(pids), 0), np.float32)
    out = []
    for i, gi in enumerate(pids.tolist()):
        for q in range(k):
            j, d = int(ids[i, q]), ds[i, q]
            if j == 0xFFFFFFFF or not np.isfinite(d):
                continue
            if j not in members:
                raise KeyError(j)
            dbits = int(np.float32(d).view(np.uint32))
            out.append((gi, j, compute_hash(sketches[gi], sketches[j], m_bits), 0, dbits))
            out.append((j, gi, compute_hash(sketches[j], sketches[gi], m_bits), 0, dbits))
    return out
