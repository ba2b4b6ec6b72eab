"""GPU parity of HashPrune with a named R-half backfill policy
(tessa_hashprune_create_backfill; SoftTier-Q3 cap 3 is the build_shear_index
binary's default) with the CPU oracle orc_hashprune_rhalf_reduce, which
tests/test_hashprune_rhalf_oracle.py pins to the reference's KATs and an
independent restatement.  Bar: every row bit-identical (primaries in
ascending hash, then backups in priority order: targets, hashes, distance
bits, counts), for record batches and segment batches, split and ordered
any way."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import hashprune as H
from test_hashprune_oracle import random_stream

pytestmark = pytest.mark.gpu

MODES = ["rhalf-soft-tier-q3", "rhalf-distance-first-q3", "rhalf-hard-tier-q3", "rhalf-hash-slot-1"]


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _want(orc, n, l_max, r, bf):
    t, hs, d, c, _ = orc.hashprune_rhalf_reduce(n, l_max, r, mode=bf.mode, hash_quota=bf.hash_quota or 0,
                                                row_cap=bf.max_backfill_per_row or 0,
                                                priority_alpha=bf.soft_tier_priority_alpha or 0.0)
    return t, hs, d, c


def _got(hp):
    t, hs, d, c = hp.slots()
    torch.cuda.synchronize()
    return (t.cpu().numpy().view(np.uint32), hs.cpu().numpy().view(np.uint16), d.cpu().numpy(),
            c.cpu().numpy().view(np.uint32))


def _same(got, want, what):
    gt, gh, gd, gc = got
    wt, wh, wd, wc = want
    bad = np.nonzero(gc != wc)[0]
    assert not len(bad), f"{what}: counts differ at points {bad[:8]} ({gc[bad[:4]]} vs {wc[bad[:4]]})"
    for p in range(len(gc)):
        n = int(gc[p])
        row_ok = (np.array_equal(gt[p, :n], wt[p, :n]) and np.array_equal(gh[p, :n], wh[p, :n])
                  and np.array_equal(gd[p, :n].view(np.uint32), wd[p, :n].view(np.uint32)))
        assert row_ok, f"{what}: point {p}: {gt[p, :n].tolist()} vs {wt[p, :n].tolist()}"
        assert np.all(gt[p, n:] == 0xFFFFFFFF), f"{what}: point {p}: unused slots"


def _segments(r, rng, dev):
    """r grouped by source, each source's run cut into pieces of 1..40
    records, the segments in random order: (records, segments) int32 tensors."""
    g = r[np.argsort(r["src"], kind="stable")]
    segs = []
    i = 0
    while i < len(g):
        j = i
        while j < len(g) and g["src"][j] == g["src"][i]:
            j += 1
        while i < j:
            m = min(j - i, int(rng.integers(1, 41)))
            segs.append((int(g["src"][i]), i & 0xFFFFFFFF, i >> 32, m))
            i += m
    sg = np.array(segs, np.uint32)[rng.permutation(len(segs))]
    rec = torch.from_numpy(np.ascontiguousarray(g).view(np.uint8).view(np.int32).reshape(-1, 4).copy()).to(dev)
    return rec, torch.from_numpy(sg.view(np.int32).copy()).to(dev)


CASES = [
    # seed, points, records, l_max, hash bits, distance levels, row cap
    (1, 6, 500, 8, 3, 7, 0),          # heavy collisions and ties; rows near full
    (2, 20, 1500, 16, 4, 50, 3),      # underfull rows with many groups
    (3, 4, 3000, 64, 4, 1000, 3),     # default R, production cap, groups of colliding targets
    (4, 30, 800, 5, 2, 3, 2),         # odd l_max
    (5, 2000, 150000, 64, 7, 4000, 3),  # ~94 records a point over 128 hashes: some rows fill mid-stream
    (6, 40, 30000, 128, 7, 5000, 0),  # two slot registers; cap floor(l_max / 2)
    (7, 300, 60000, 256, 6, 20000, 0),  # four slot registers, 64 groups, cap 128
]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("seed,num_points,n,l_max,hash_bits,levels,row_cap", CASES)
def test_record_batches_match_oracle(gpu, orc, mode, seed, num_points, n, l_max, hash_bits, levels, row_cap):
    rng = np.random.default_rng(seed)
    r = random_stream(rng, num_points, n, hash_bits, levels)
    extra = r[rng.integers(0, n, n // 4)].copy()  # the same targets at other distances
    extra["dist"] = rng.integers(0, levels, len(extra)).astype(np.float32) * np.float32(0.25)
    r = np.concatenate([r, extra])
    bf = H.HashPruneBackfill(mode, None, row_cap or None, 1.02 if mode == "rhalf-soft-tier-q3" else None)
    want = _want(orc, num_points, l_max, r, bf)
    with H.HashPruneReducer(num_points, l_max, backfill=bf) as hp:
        perm = rng.permutation(len(r))
        for part in np.array_split(r[perm], 3):
            hp.insert(part)
        _same(_got(hp), want, f"{mode} seed {seed} records")
        hp.clear()
        rec, segs = _segments(r, rng, gpu)
        half = segs.shape[0] // 2
        hp.insert_segments(rec, segs[:half])
        hp.insert_segments(rec, segs[half:])
        _same(_got(hp), want, f"{mode} seed {seed} segments")
    if seed in (2, 3, 5):
        assert int(np.sum(want[3])) > 0


def test_default_policy_and_mixed_batches(gpu, orc):
    # zero fields take the reference's defaults (quota 3, alpha 1.1, cap
    # floor(l_max / 2)); record and segment batches merge into one state
    rng = np.random.default_rng(31)
    r = random_stream(rng, 300, 40000, 6, 700)  # ~57 hashes a point: 179 rows fill, 121 take backups
    bf = H.HashPruneBackfill("rhalf-soft-tier-q3")
    want = _want(orc, 300, 56, r, bf)
    a, b = r[: len(r) // 2], r[len(r) // 2:]
    with H.HashPruneReducer(300, 56, backfill=bf) as hp:
        rec, segs = _segments(b, rng, gpu)
        hp.insert(a)
        hp.insert_segments(rec, segs)
        _same(_got(hp), want, "mixed batches")
    _, _, _, c0 = orc.hashprune_reduce(300, 56, r)
    assert np.any(c0 == 56) and np.any(want[3] > c0)


def test_kat_rows_on_gpu(gpu, orc):
    # the reference KATs (hash_prune.rs:2468-2487 at l_max 4, two points of
    # one batch; :2505-2527 at l_max 8, in a reducer of its own)
    a2_in, a2_out = float(np.float32(0.90) ** 2), float(np.float32(0.95) ** 2)
    rows = []
    for src, a2 in ((0, a2_in), (1, a2_out)):
        for t, h, d in ((10, 10, 0.25), (101, 10, 0.30), (102, 10, a2), (20, 20, 0.25), (201, 20, 1.00)):
            rows.append((src, t, h, 0, d))
    r = np.array(rows, orc.EDGE_DTYPE)
    bf = H.HashPruneBackfill("rhalf-soft-tier-q3")
    with H.HashPruneReducer(2, 4, backfill=bf) as hp:
        hp.insert(r)
        t, hs, d, c = _got(hp)
    assert sorted(t[0, :c[0]].tolist()[2:]) == [101, 102]
    assert sorted(t[1, :c[1]].tolist()[2:]) == [101, 201]
    c2 = [(10, 1, 1.0), (11, 1, 1.1), (12, 1, 1.2), (20, 2, 0.8), (21, 2, 1.0), (30, 3, 0.7)]
    r = np.array([(0, t_, h_, 0, d_) for t_, h_, d_ in c2], orc.EDGE_DTYPE)
    with H.HashPruneReducer(1, 8, backfill=bf) as hp:
        hp.insert(r)
        t, hs, d, c = _got(hp)
    assert t[0, :c[0]].tolist() == [10, 20, 30, 21, 11, 12]


def test_policy_off_equals_plain_reservoir(gpu, orc):
    rng = np.random.default_rng(5)
    r = random_stream(rng, 50, 5000, 4, 100)
    with H.HashPruneReducer(50, 16, backfill=H.HashPruneBackfill("off")) as hp:
        assert hp.backfill is None
        hp.insert(r)
        t, hs, d, c = _got(hp)
    wt, wh, wd, wc = orc.hashprune_reduce(50, 16, r)
    assert np.array_equal(t, wt) and np.array_equal(c, wc)
