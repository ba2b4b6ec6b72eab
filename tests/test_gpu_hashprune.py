"""GPU parity of the HashPrune reservoirs (tessa_hashprune_*) with the CPU
oracle's restatement of HashPruneReservoir insertion fed record by record
(spill_hashprune.rs:2686-2719).  Bar: every point's slots bit-identical
(targets, hashes, distance bits, counts, slot order)."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import _native as N
from shear_amd import edges as E
from shear_amd import hashprune as H
from test_gpu_edges import _batches, _leaf_case, _oracle_records
from test_hashprune_oracle import random_stream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _gpu_slots(hp):
    t, hs, d, c = hp.slots()
    torch.cuda.synchronize()
    return (t.cpu().numpy().view(np.uint32), hs.cpu().numpy().view(np.uint16), d.cpu().numpy(),
            c.cpu().numpy().view(np.uint32))


def _same(got, want, what=""):
    gt, gh, gd, gc = got
    wt, wh, wd, wc = want
    assert np.array_equal(gc, wc), f"{what} counts differ at points {np.nonzero(gc != wc)[0][:8]}"
    assert np.array_equal(gt, wt), f"{what} targets differ at points {np.nonzero(np.any(gt != wt, 1))[0][:8]}"
    assert np.array_equal(gh, wh), what
    assert np.array_equal(gd.view(np.uint32), wd.view(np.uint32)), what


@pytest.mark.parametrize("seed,num_points,n,l_max,hash_bits,levels", [
    (1, 5, 400, 4, 3, 7),          # heavy hash collisions and distance ties
    (2, 17, 2000, 8, 5, 50),
    (3, 3, 3000, 64, 12, 1000),     # > 512 records per point: several merge rounds
    (4, 40, 5000, 3, 2, 3),
    (5, 1000, 60000, 64, 12, 4000),  # default l_max and m_hash_bits
    (6, 7, 9000, 256, 12, 100000),  # largest l_max
    (7, 300, 2000, 1, 1, 2),
    (8, 20, 4000, 32, 12, 500),      # 129..256 candidates per point, in registers
    (9, 20, 4000, 200, 12, 500),
    (10, 60, 9000, 64, 8, 300),      # 256 hashes: many collisions at 150 candidates
    (11, 30, 12000, 64, 12, 3000),   # 257..512 candidates per point: the LDS merge
    (12, 25, 10000, 256, 12, 50000),  # the same band, more than l_max = 256 hashes kept
    (13, 30, 12000, 32, 6, 100),     # the band with 64 hashes: heavy collisions and ties
])
def test_random_streams_match_oracle(gpu, orc, seed, num_points, n, l_max, hash_bits, levels):
    rng = np.random.default_rng(seed)
    r = random_stream(rng, num_points, n, hash_bits, levels)
    with H.HashPruneReducer(num_points, l_max) as hp:
        hp.insert(r)
        _same(_gpu_slots(hp), orc.hashprune_reduce(num_points, l_max, r), f"seed {seed}")


def test_batches_in_any_split_and_order(gpu, orc):
    rng = np.random.default_rng(21)
    r = random_stream(rng, 50, 20000, 6, 300)
    r = np.concatenate([r, r[:3000]])  # the same edge from several leaves
    want = orc.hashprune_reduce(50, 16, r)
    with H.HashPruneReducer(50, 16) as hp:
        perm = rng.permutation(len(r))
        cuts = np.sort(rng.choice(len(r), 6, replace=False))
        for part in np.split(r[perm], cuts):
            hp.insert(part)
        _same(_gpu_slots(hp), want, "split batches")
        hp.clear()
        t, c = hp.neighbors()
        torch.cuda.synchronize()
        assert int(c.sum()) == 0 and bool(torch.all(t == -1))
        hp.insert(r[::-1].copy())  # reused after clear
        _same(_gpu_slots(hp), want, "after clear")


def test_second_batch_lands_in_the_register_band(gpu, orc):
    # full reservoirs (64 slots) + ~300 new records: slots + records in 257..512
    rng = np.random.default_rng(14)
    r = random_stream(rng, 40, 30000, 12, 4000)
    want = orc.hashprune_reduce(40, 64, r)
    with H.HashPruneReducer(40, 64) as hp:
        for part in np.array_split(r, 2):
            hp.insert(part)
        _same(_gpu_slots(hp), want, "two batches")


def test_hub_point_and_empty_batches(gpu, orc):
    rng = np.random.default_rng(5)
    r = random_stream(rng, 4, 5000, 12, 2000)
    r["src"][: 4000] = 2  # one point with thousands of candidates in one batch
    with H.HashPruneReducer(4, 64) as hp:
        hp.insert(np.zeros(0, E.EDGE_RECORD_DTYPE))
        hp.insert(r)
        hp.insert(np.zeros(0, E.EDGE_RECORD_DTYPE))
        _same(_gpu_slots(hp), orc.hashprune_reduce(4, 64, r), "hub")


def test_records_from_the_leaf_operator(gpu, orc):
    # leaf top-k -> edge records on the GPU -> HashPrune reservoirs, against the
    # oracle fed with the oracle's own records for the same leaves
    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, [33, 100, 257, 1024, 300, 2], 48, 32, 3)
    rec, n = E.emit_edge_records(g, lay, 32, ids, d, torch.from_numpy(sk).to(gpu), 12)
    want_rec = _oracle_records(orc, _batches(gids, members, offs, sizes, ids, d, 32), sk, 12)
    num_points = int(gids.max()) + 1
    with H.HashPruneReducer(num_points, 64) as hp:
        hp.insert(rec, n)
        _same(_gpu_slots(hp), orc.hashprune_reduce(num_points, 64, want_rec), "leaf records")
    lists = H.reduce_spill_records_ordered(num_points, 64, want_rec)
    t, _, _, c = orc.hashprune_reduce(num_points, 64, want_rec)
    assert lists == [t[p, :c[p]].tolist() for p in range(num_points)]


def test_out_of_range_source_is_rejected(gpu, orc):
    rng = np.random.default_rng(3)
    r = random_stream(rng, 10, 500, 5, 40)
    bad = r.copy()
    bad["src"][123] = 10
    with H.HashPruneReducer(10, 8) as hp:
        with pytest.raises(N.TessaError, match=r"outside shard range \[0, 10\)"):
            hp.insert(bad)
        # the batch's valid records were merged
        keep = np.ones(len(bad), bool)
        keep[123] = False
        _same(_gpu_slots(hp), orc.hashprune_reduce(10, 8, bad[keep]), "valid part")


def test_l_max_limits(gpu):
    with pytest.raises(N.TessaError, match="l_max=257"):
        H.HashPruneReducer(4, 257)
    with pytest.raises(N.TessaError, match="l_max must be > 0"):
        H.HashPruneReducer(4, 0)


def test_spill_round_trip_of_device_records(gpu, orc, tmp_path):
    # device records -> spill part files + manifest -> read back -> reservoirs
    # identical to merging the device records directly
    from shear_amd import spill as SP

    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, [100, 257, 1024, 64], 32, 16, 4)
    rec, n = E.emit_edge_records(g, lay, 16, ids, d, torch.from_numpy(sk).to(gpu), 12)
    num_points = int(gids.max()) + 1
    SP.write_spill_artifacts(tmp_path / "cand", rec, n, shard_points=max(1, num_points // 3), segment_records=700)
    back = SP.read_spill_artifacts(tmp_path / "cand", shard_points=max(1, num_points // 3))
    assert len(back) == n
    with H.HashPruneReducer(num_points, 64) as a, H.HashPruneReducer(num_points, 64) as b:
        a.insert(rec, n)
        b.insert(back)
        _same(_gpu_slots(b), _gpu_slots(a), "spilled records")
