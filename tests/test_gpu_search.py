"""GPU parity of the greedy search (tessa_graph_search) with the CPU oracle's
restatement of greedy_search (shear-core/src/algorithm/search/search.rs:
137-233, neighbour queue model/neighbor/neighbor_priority_queue.rs:50-85).
Bar: ids, distance bits and distance-evaluation counts identical per query."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import _native as N
from shear_amd import graph as G
from shear_amd import hashprune as H
from test_hashprune_oracle import random_stream
from test_search_oracle import brute_force, complete_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def random_graph(rng, n, stride, extra_junk=True):
    t = rng.integers(0, n, (n, stride)).astype(np.uint32)
    c = rng.integers(0, stride + 1, n).astype(np.uint32)
    if extra_junk:
        t[rng.random((n, stride)) < 0.02] = n + 5  # out-of-range ids are skipped
        c[rng.random(n) < 0.05] = stride + 9      # counts clip to the stride
    return t, c


def _run(gpu, x, t, c, start, q, L, K, misalign=False):
    xd = torch.from_numpy(x).to(gpu)
    if misalign:  # 4-byte aligned rows only: the scalar distance path
        buf = torch.empty(x.size + 1, dtype=torch.float32, device=gpu)
        buf[1:] = xd.reshape(-1)
        xd = buf[1:].view(x.shape)
    ids, d, cm = G.greedy_search(xd, torch.from_numpy(t.view(np.int32)).to(gpu),
                                 torch.from_numpy(c.astype(np.int32)).to(gpu), start, torch.from_numpy(q).to(gpu), L, K)
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), cm.cpu().numpy().view(np.uint32)


def _same(got, want, what):
    gi, gd, gc = got
    wi, wd, wc = want
    bad = np.nonzero(np.any(gi != wi, 1) | np.any(gd.view(np.uint32) != wd.view(np.uint32), 1) | (gc != wc))[0]
    assert len(bad) == 0, f"{what}: queries {bad[:8]} differ, e.g. got {gi[bad[0]][:8]} want {wi[bad[0]][:8]}"


@pytest.mark.parametrize("seed,n,dim,stride,L,K,nq", [
    (1, 500, 16, 12, 20, 10, 64),
    (2, 3000, 128, 32, 64, 10, 200),
    (3, 2000, 7, 24, 100, 50, 33),      # dim not a multiple of 4: scalar loads
    (4, 1000, 32, 150, 256, 256, 40),   # rows of 150: three chunks per expansion, largest L
    (5, 800, 3, 8, 1, 1, 17),
    (6, 300000, 8, 16, 32, 10, 2000),   # 1 GiB of tags holds 894 slots: queries reuse a slot's tags
])
def test_random_graphs_match_oracle(gpu, orc, seed, n, dim, stride, L, K, nq):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    t, c = random_graph(rng, n, stride)
    start = int(rng.integers(0, n))
    _same(_run(gpu, x, t, c, start, q, L, K), orc.greedy_search(x, t, c, start, q, L, K), f"seed {seed}")


def test_unaligned_rows_use_the_scalar_path(gpu, orc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((700, 12)).astype(np.float32)
    q = rng.standard_normal((50, 12)).astype(np.float32)
    t, c = random_graph(rng, 700, 16)
    want = orc.greedy_search(x, t, c, 3, q, 40, 10)
    _same(_run(gpu, x, t, c, 3, q, 40, 10, misalign=True), want, "misaligned")
    _same(_run(gpu, x, t, c, 3, q, 40, 10), want, "aligned")


def test_complete_graph_is_exact(gpu):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((120, 20)).astype(np.float32)
    q = rng.standard_normal((30, 20)).astype(np.float32)
    t, c = complete_graph(120)
    ids, d, cm = _run(gpu, x, t, c, 0, q, 128, 10)
    want_ids, want_d = brute_force(x, q, 10)
    assert np.array_equal(ids, want_ids) and np.array_equal(d.view(np.uint32), want_d.view(np.uint32))
    assert np.all(cm == 119)


def test_ties_duplicates_and_dead_ends(gpu, orc):
    rng = np.random.default_rng(2)
    x = rng.integers(0, 3, (400, 4)).astype(np.float32)  # many equal distances: ties by id
    q = rng.integers(0, 3, (40, 4)).astype(np.float32)
    t, c = random_graph(rng, 400, 20)
    t[:, 10:] = t[:, :10]  # every id twice in its row
    c[::7] = 0  # rows with no neighbours
    for start in (0, 1, 399):
        _same(_run(gpu, x, t, c, start, q, 30, 30), orc.greedy_search(x, t, c, start, q, 30, 30), f"start {start}")


def test_hashprune_graph_search(gpu, orc):
    # reservoirs -> neighbour table -> search, the table taken from the device
    rng = np.random.default_rng(8)
    n, dim = 600, 24
    x = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((64, dim)).astype(np.float32)
    r = random_stream(rng, n, 40000, 12, 5000)
    r["dst"] = r["dst"] % n
    with H.HashPruneReducer(n, 32) as hp:
        hp.insert(r)
        tt, cc = hp.neighbors()
        got = G.greedy_search(torch.from_numpy(x).to(gpu), tt, cc, 0, torch.from_numpy(q).to(gpu), 50, 10)
        torch.cuda.synchronize()
        t_host, c_host = tt.cpu().numpy().view(np.uint32), cc.cpu().numpy().view(np.uint32)
    got = tuple(a.cpu().numpy() for a in got)
    got = (got[0].view(np.uint32), got[1], got[2].view(np.uint32))
    _same(got, orc.greedy_search(x, t_host, c_host, 0, q, 50, 10), "hashprune graph")


def test_argument_errors(gpu):
    x = torch.zeros((10, 4), device=gpu)
    t = torch.zeros((10, 2), dtype=torch.int32, device=gpu)
    c = torch.zeros(10, dtype=torch.int32, device=gpu)
    with pytest.raises(N.TessaError, match="Set L: 5 to a value of at least K: 10"):
        G.greedy_search(x, t, c, 0, x[:2], 5, 10)
    with pytest.raises(N.TessaError, match="L=257"):
        G.greedy_search(x, t, c, 0, x[:2], 257, 10)
    with pytest.raises(N.TessaError, match="start 10"):
        G.greedy_search(x, t, c, 10, x[:2], 20, 10)
    ids, _, cm = G.greedy_search(x, t, c, 4, x[:3], 4, 2)  # only the start is reachable
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [[4, -1]] * 3 and cm.cpu().tolist() == [0] * 3



@pytest.mark.parametrize("seed,n,dim,stride,L,K,nq", [
    (11, 4000, 128, 32, 64, 10, 200),   # dim a multiple of 16: 16 codes per load
    (12, 1500, 20, 16, 40, 10, 60),     # dim 20 (padded to 32): the scalar path
])
def test_sq8_rows_match_oracle_on_dequantized_vectors(gpu, orc, seed, n, dim, stride, L, K, nq):
    """tessa_graph_search_sq8 equals the oracle's search over the dequantized
    rows scale * code (f32 products, rounded), bit for bit."""
    from shear_amd import tessa as T

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    t, c = random_graph(rng, n, stride)
    sq8 = T.quantize_sq_int8_matrix(torch.from_numpy(x).to(gpu))
    codes = sq8.codes.cpu().numpy()[:, :dim].astype(np.float32)
    xhat = (sq8.scales.cpu().numpy()[:, None] * codes).astype(np.float32)
    want = orc.greedy_search(xhat, t, c, 5, q, L, K)
    ids, d, cm = G.greedy_search_sq8(sq8, torch.from_numpy(t.view(np.int32)).to(gpu),
                                     torch.from_numpy(c.astype(np.int32)).to(gpu), 5, torch.from_numpy(q).to(gpu), L, K)
    torch.cuda.synchronize()
    _same((ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), cm.cpu().numpy().view(np.uint32)), want,
          f"sq8 seed {seed}")
