"""Source-grouped record emission (tessa_emit_edge_segments) and the HashPrune
segment insert (tessa_hashprune_insert_segments).

  * per leaf, the grouped records are the reference-order records
    (tessa_emit_edge_records) as a multiset; every segment's records carry
    its source, the segments tile the records, one per member row;
  * the reservoirs after inserting by segments equal those after inserting
    the records (C2-shaped leaves, and replicated points across leaves with
    hub sources that take the LDS merge), and equal the oracle's;
  * tessa_emit_edge_segments_unique writes, per leaf, the reference-order
    multiset less exactly one copy of each mutual pair's repeated record
    (found here from the top-k lists on the host), with no gaps, and the
    reservoirs it feeds equal the oracle's over every record."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev_u32, require_gpu, to_dev_sq8
from shear_amd import edges as E
from shear_amd import hashprune as H
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu


def _leaves(orc, n_points, leaf_sizes, dim, seed, replicate=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_points, dim)).astype(np.float32)
    codes, scales, norms = orc.quantize(x)
    members, offs, counts = [], [], []
    at = 0
    for n in leaf_sizes:
        rows = np.sort(rng.choice(n_points, n, replace=False)).astype(np.uint32)
        members.append(rows)
        offs.append(at)
        counts.append(n)
        at += n
    return codes, scales, norms, np.concatenate(members), np.array(offs), np.array(counts)


def _run(orc, gpu, n_points, leaf_sizes, dim, seed, k=32, m_bits=12, unique=False, full=False):
    codes, scales, norms, members, offs, counts = _leaves(orc, n_points, leaf_sizes, dim, seed)
    sq8 = to_dev_sq8(codes, scales, norms, dim)
    gids = dev_u32(np.arange(n_points))
    lay = T.LeafLayouts.from_host(members, offs, counts, k, gpu)
    ids, d, _ = T.leaf_topk(sq8, gids, lay, k)
    rng = np.random.default_rng(seed + 1)
    sk = torch.from_numpy(rng.standard_normal((n_points, m_bits)).astype(np.float32)).to(gpu)
    lro = torch.zeros(len(leaf_sizes) + 1, dtype=torch.int64, device=gpu)
    rec, cnt = E.emit_edge_records(gids, lay, k, ids, d, sk, m_bits, leaf_record_offsets=lro)
    grec, gcnt, segs, nseg = E.emit_edge_segments(gids, lay, k, ids, d, sk, m_bits, unique=unique)
    if full:
        return rec, cnt, grec, gcnt, segs, nseg, counts, members, offs, ids, d, lro
    return rec, cnt, grec, gcnt, segs, nseg, counts


def _sorted_records(r):
    v = np.ascontiguousarray(r).view(np.uint8).reshape(-1, 16).view("V16").ravel()
    return np.sort(v)


@pytest.mark.parametrize("n_points,leaf_sizes,dim", [
    (8192, [1024] * 8, 128),                      # C2-shaped: each point in one leaf
    (3000, [700, 2048, 33, 2, 1, 1500, 900], 64),  # ragged leaves, replicated points, a one-row leaf
])
def test_grouped_records_and_segments(gpu_dev, orc, n_points, leaf_sizes, dim):
    rec, cnt, grec, gcnt, segs, nseg, counts = _run(orc, gpu_dev, n_points, leaf_sizes, dim, 5)
    assert cnt == gcnt
    assert nseg == int(np.sum(counts))
    a = E.records_to_numpy(rec, cnt)
    b = E.records_to_numpy(grec, gcnt)
    assert np.array_equal(_sorted_records(a), _sorted_records(b)), "grouped records differ as a multiset"
    sg = segs[:nseg].cpu().numpy().view(np.uint32)
    first = sg[:, 1].astype(np.uint64) | (sg[:, 2].astype(np.uint64) << 32)
    order = np.argsort(first, kind="stable")
    covered = 0
    for i in order:
        src, c = int(sg[i, 0]), int(sg[i, 3])
        f = int(first[i])
        if c == 0:
            continue
        assert f == covered, "segments must tile the records"
        assert np.all(b["src"][f:f + c] == src)
        covered += c
    assert covered == gcnt


def _tiles(segs, nseg, n_records, recs):
    """Segments tile records [0, n_records) and carry their records' source."""
    sg = segs[:nseg].cpu().numpy().view(np.uint32)
    first = sg[:, 1].astype(np.uint64) | (sg[:, 2].astype(np.uint64) << 32)
    covered = 0
    for i in np.argsort(first, kind="stable"):
        c = int(sg[i, 3])
        if c == 0:
            continue
        assert int(first[i]) == covered, "segments must tile the records"
        assert np.all(recs["src"][covered:covered + c] == sg[i, 0])
        covered += c
    assert covered == n_records
    return sg, first


@pytest.mark.parametrize("n_points,leaf_sizes,dim,k", [
    (8192, [1024] * 8, 128, 32),                       # C2-shaped
    (3000, [700, 2048, 33, 2, 1, 1500, 900], 64, 32),   # ragged leaves, replicated points, a one-row leaf
    (600, [20, 300, 7, 250], 16, 10),                   # k_eff below k, k not a multiple of 4
])
def test_unique_segments_drop_only_mutual_repeats(gpu_dev, orc, n_points, leaf_sizes, dim, k):
    rec, cnt, urec, ucnt, segs, nseg, counts, members, offs, ids, d, lro = _run(
        orc, gpu_dev, n_points, leaf_sizes, dim, 5, k=k, unique=True, full=True)
    a = E.records_to_numpy(rec, cnt)
    u = E.records_to_numpy(urec, ucnt)
    sg, first = _tiles(segs, nseg, ucnt, u)
    lro = lro.cpu().numpy()
    ids_h = ids.cpu().numpy().view(np.uint32)
    d_h = d.cpu().numpy().view(np.uint32)
    seg0, dropped_total = 0, 0
    for leaf, n in enumerate(counts):
        n = int(n)
        m = members[offs[leaf]:offs[leaf] + n].astype(np.uint32)  # global id = row (sorted, distinct)
        kl = min(k, n - 1) if n > 1 else 0
        start = int(offs[leaf]) * k
        li = ids_h[start:start + n * k].reshape(n, k)[:, :kl]
        ld = d_h[start:start + n * k].reshape(n, k)[:, :kl]
        want = a[lro[leaf]:lro[leaf + 1]]
        # this leaf's kept records: its rows' segments
        got = np.concatenate([u[int(first[i]):int(first[i]) + int(sg[i, 3])] for i in range(seg0, seg0 + n)]
                             + [u[:0]])
        seg0 += n
        # the slots (r, q) whose target row lists m[r] at the same distance
        drop = []
        if kl:
            c = np.searchsorted(m, li)
            assert np.all(m[c] == li)
            mutual = (li[c] == m[:, None, None]) & (ld[c] == ld[:, :, None])  # [r, q, slot of c's list]
            rr, qq = np.nonzero(mutual.any(axis=2))
            drop = [(int(li[r, q]), int(m[r]), int(ld[r, q])) for r, q in zip(rr, qq)]
        dropped_total += len(drop)
        # want less one copy of each repeated record equals what was kept
        key = {}
        for i, (s_, t_, db) in enumerate(zip(want["src"], want["dst"], want["dist"].view(np.uint32))):
            key.setdefault((int(s_), int(t_), int(db)), []).append(i)
        keep = np.ones(len(want), bool)
        for dk in drop:
            copies = key[dk]
            assert len(copies) == 2, f"leaf {leaf}: a mutual pair's record appears {len(copies)} times"
            keep[copies.pop()] = False
        assert np.array_equal(_sorted_records(want[keep]), _sorted_records(got)), f"leaf {leaf}"
    assert ucnt == cnt - dropped_total and dropped_total > 0


@pytest.fixture(scope="module")
def gpu_dev():
    return require_gpu()


@pytest.mark.parametrize("unique", [False, True])
@pytest.mark.parametrize("n_points,leaf_sizes,dim,l_max", [
    (8192, [1024] * 8, 128, 64),
    (1500, [1400, 1400, 1300, 900, 1450, 1200], 32, 16),  # points in up to six leaves: large merges
])
def test_segment_insert_equals_record_insert(gpu_dev, orc, n_points, leaf_sizes, dim, l_max, unique):
    rec, cnt, grec, gcnt, segs, nseg, _ = _run(orc, gpu_dev, n_points, leaf_sizes, dim, 9, unique=unique)
    with H.HashPruneReducer(n_points, l_max, gpu_dev) as a, H.HashPruneReducer(n_points, l_max, gpu_dev) as b:
        a.insert(rec, cnt)
        b.insert_segments(grec, segs, nseg)
        # a second batch into the same reservoirs (existing slots + new segments)
        a.insert(rec, cnt)
        b.insert_segments(grec, segs, nseg)
        ta, _, da, ca = a.slots()
        tb, _, db, cb = b.slots()
    assert torch.equal(ca, cb) and torch.equal(ta, tb) and torch.equal(da, db)
    wt, _, _, wc = orc.hashprune_reduce(n_points, l_max, E.records_to_numpy(rec, cnt))
    assert np.array_equal(cb.cpu().numpy().view(np.uint32), wc)
    tbn = tb.cpu().numpy().view(np.uint32)
    for p in range(n_points):
        assert np.array_equal(tbn[p, : wc[p]], wt[p, : wc[p]])


def _random_segments(rng, r, max_seg):
    """The records of stream ``r`` grouped by source and cut into segments of
    1..max_seg records of one source, in random order."""
    g = r[np.argsort(r["src"], kind="stable")]
    src = g["src"].astype(np.int64)
    cut = np.zeros(len(g) + 1, bool)
    cut[0] = cut[-1] = True
    cut[1:-1] = src[1:] != src[:-1]
    pos, starts = 0, []
    for b in np.nonzero(cut[1:])[0] + 1:  # source runs [pos, b)
        while pos < b:
            starts.append(pos)
            pos += int(rng.integers(1, max_seg + 1))
        pos = b
    starts = np.array(starts, np.int64)
    ends = np.append(starts[1:], len(g))
    bounds = np.nonzero(cut)[0]
    ends = np.minimum(ends, bounds[np.searchsorted(bounds, starts, side="right")])
    segs = np.zeros((len(starts), 4), np.uint32)
    segs[:, 0] = src[starts]
    segs[:, 1] = starts & 0xFFFFFFFF
    segs[:, 2] = starts >> 32
    segs[:, 3] = ends - starts
    segs = segs[rng.permutation(len(segs))]
    return g, segs


@pytest.mark.parametrize("seed,num_points,n,l_max,hash_bits,levels,max_seg", [
    (1, 5, 400, 4, 3, 7, 3),           # heavy hash collisions and distance ties
    (2, 17, 2000, 8, 5, 50, 40),
    (3, 3, 3000, 64, 12, 1000, 2),     # ~1000 records per source in > 64 segments of 1..2
    (4, 40, 5000, 3, 2, 3, 9),
    (5, 1000, 60000, 64, 12, 4000, 70),  # default l_max and m_hash_bits
    (6, 7, 9000, 256, 12, 100000, 300),  # largest l_max
    (7, 300, 2000, 1, 1, 2, 5),
    (8, 20, 4000, 32, 12, 500, 17),
    (9, 20, 4000, 200, 12, 500, 64),
    (10, 60, 9000, 64, 8, 300, 33),     # 256 hashes: many collisions
    (11, 30, 12000, 64, 12, 3000, 128),
    (12, 25, 10000, 256, 12, 50000, 1),  # 400 one-record segments per source
    (13, 30, 12000, 32, 6, 100, 6),     # 64 hashes: heavy collisions and ties
    (14, 2000, 200000, 128, 12, 100000, 40),
    (15, 500, 100000, 100, 10, 1000, 25),
])
def test_random_segments_match_oracle(gpu_dev, orc, seed, num_points, n, l_max, hash_bits, levels, max_seg):
    """Random streams (the record-path cases) through the segment insert, in
    two batches of segments: slot for slot the oracle's reservoirs."""
    from test_gpu_hashprune import _gpu_slots, _same
    from test_hashprune_oracle import random_stream

    rng = np.random.default_rng(seed)
    r = random_stream(rng, num_points, n, hash_bits, levels)
    g, segs = _random_segments(rng, r, max_seg)
    recs = torch.from_numpy(np.ascontiguousarray(g).view(np.uint8).view(np.int32).reshape(-1, 4).copy()).to(gpu_dev)
    half = len(segs) // 2
    with H.HashPruneReducer(num_points, l_max, gpu_dev) as hp:
        for part in (segs[:half], segs[half:]):
            hp.insert_segments(recs, torch.from_numpy(part.view(np.int32).copy()).to(gpu_dev))
        _same(_gpu_slots(hp), orc.hashprune_reduce(num_points, l_max, r), f"seed {seed}")
