"""The leaf top-k entry point that allocates nothing (tessa_leaf_topk_noalloc),
through the C ABI: two calls in a row, the second smaller, each identical bit
for bit to tessa_leaf_topk on the same inputs (and the small one to the CPU
oracle); a batch beyond the static scratch is rejected before any work."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_same, dev_u32, require_gpu, to_dev_sq8
from shear_amd import _native as N
from shear_amd import datagen
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu

MAX_ROWS = 65536  # the entry point's limit on leaf_count * max_leaf_rows


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _leaves(sizes):
    sizes = np.asarray(sizes, np.int64)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    return np.arange(int(sizes.sum()), dtype=np.uint32), offs, sizes


def _both(sq8, gids, members, offs, sizes, k):
    lay = T.LeafLayouts.from_host(members, offs, sizes, k)
    g = dev_u32(gids)
    ref_ids, ref_d, ref_ctr = T.leaf_topk(sq8, g, lay, k, executor=N.EXEC_MFMA)
    ids, d, ctr = T.leaf_topk(sq8, g, lay, k, executor=N.EXEC_MFMA, no_alloc=True)
    torch.cuda.synchronize()
    T.raise_on_overflow(ref_ctr, "leaf top-k")
    T.raise_on_overflow(ctr, "leaf top-k (no allocation)")
    ids_h, d_h = ids.cpu().numpy().view(np.uint32), d.cpu().numpy()
    assert_same(ids_h, d_h, ref_ids.cpu().numpy().view(np.uint32), ref_d.cpu().numpy(), "no-alloc vs allocating")
    assert ctr.cpu().numpy()[N.C_LEAF_ROWS] == ref_ctr.cpu().numpy()[N.C_LEAF_ROWS] == int(np.sum(sizes))
    return ids_h, d_h


def test_noalloc_matches_allocating_entry_on_two_calls(gpu, orc):
    # first call: 60 leaves x 1,024 rows x 768-d (61,440 rows, 240 work items,
    # so several filter/select batches run through the one static log)
    n1 = 60 * 1024
    x1 = datagen.gmm_numpy(n1, 768, 60, 0.3, 31)
    c1, s1, nn1 = orc.quantize(x1)
    g1 = np.random.default_rng(31).permutation(1 << 24)[:n1].astype(np.uint32)
    m1, o1, z1 = _leaves([1024] * 60)
    _both(to_dev_sq8(c1, s1, nn1, 768), g1, m1, o1, z1, 32)

    # second call, smaller: ragged leaves (including 1- and 2-row ones) in 96-d,
    # also checked against the oracle
    sizes = [700, 1, 2, 33, 256, 257, 513, 64]
    n2 = int(np.sum(sizes))
    x2 = datagen.gmm_numpy(n2, 96, 6, 0.3, 32)
    c2, s2, nn2 = orc.quantize(x2)
    g2 = np.random.default_rng(32).permutation(1 << 24)[:n2].astype(np.uint32)
    m2, o2, z2 = _leaves(sizes)
    ids, d = _both(to_dev_sq8(c2, s2, nn2, 96), g2, m2, o2, z2, 16)
    want_ids, want_d = orc.leaf_topk(c2, s2, nn2, g2, m2, o2, sizes, 16)
    assert_same(ids, d, want_ids, want_d, "no-alloc vs oracle")


def test_noalloc_rejects_batches_beyond_its_scratch(gpu, orc):
    x = datagen.gmm_numpy(2048, 32, 4, 0.3, 33)
    c, s, nn = orc.quantize(x)
    sq8 = to_dev_sq8(c, s, nn, 32)
    members, offs, sizes = _leaves([1024, 1024])
    lay = T.LeafLayouts.from_host(members, offs, sizes, 8)
    lay.max_leaf_rows = MAX_ROWS  # 2 leaves x 65,536 rows bound: over the limit
    with pytest.raises(RuntimeError, match="no-allocation limit"):
        T.leaf_topk(sq8, dev_u32(np.arange(2048)), lay, 8, executor=N.EXEC_MFMA, no_alloc=True)


def test_noalloc_call_captured_in_a_graph(gpu, orc):
    """A warmed-up call captured into a HIP graph (torch.cuda.graph), replayed
    three times with eager work and synchronisation between the replays:
    every replay equals the eager call bit for bit."""
    sizes = [1024, 700, 1, 300, 1024]
    n = int(np.sum(sizes))
    x = datagen.gmm_numpy(n, 768, 5, 0.3, 34)
    c, s, nn = orc.quantize(x)
    sq8 = to_dev_sq8(c, s, nn, 768)
    gids = dev_u32(np.random.default_rng(34).permutation(1 << 24)[:n].astype(np.uint32))
    members, offs, z = _leaves(sizes)
    lay = T.LeafLayouts.from_host(members, offs, z, 32)
    want_ids, want_d, _ = T.leaf_topk(sq8, gids, lay, 32, executor=N.EXEC_MFMA, no_alloc=True)  # warm-up
    torch.cuda.synchronize()
    want_ids, want_d = want_ids.clone(), want_d.clone()
    out_ids = torch.empty_like(want_ids)
    out_d = torch.empty_like(want_d)
    ctr = torch.zeros(N.COUNTER_WORDS, dtype=torch.int64, device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctr.zero_()
        T.leaf_topk(sq8, gids, lay, 32, executor=N.EXEC_MFMA, out_ids=out_ids, out_dists=out_d, counters=ctr,
                    no_alloc=True)
    for rep in range(3):
        out_ids.fill_(-1)
        out_d.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        T.raise_on_overflow(ctr, "captured leaf top-k")
        assert int(ctr[N.C_LEAF_ROWS]) == n, rep
        assert_same(out_ids.cpu().numpy().view(np.uint32), out_d.cpu().numpy(),
                    want_ids.cpu().numpy().view(np.uint32), want_d.cpu().numpy(), f"graph replay {rep}")


def test_noalloc_exact_executor_takes_any_batch(gpu, orc):
    """The exact executor needs no scratch: a batch above the MFMA limit runs
    and matches the oracle."""
    x = datagen.gmm_numpy(2048, 32, 4, 0.3, 35)
    c, s, nn = orc.quantize(x)
    sq8 = to_dev_sq8(c, s, nn, 32)
    members, offs, sizes = _leaves([1024, 1024])
    lay = T.LeafLayouts.from_host(members, offs, sizes, 8)
    lay.max_leaf_rows = MAX_ROWS  # leaf_count * max_leaf_rows above the MFMA limit
    gids = np.arange(2048, dtype=np.uint32)
    ids, d, ctr = T.leaf_topk(sq8, dev_u32(gids), lay, 8, executor=N.EXEC_EXACT, no_alloc=True)
    torch.cuda.synchronize()
    want_ids, want_d = orc.leaf_topk(c, s, nn, gids, members, offs, sizes, 8)
    assert_same(ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), want_ids, want_d, "exact no-alloc")
