"""BASELINE configs[0] (C1) end to end: 200,000 x 128 mixture points (64
components, centres N(0, I), sigma 0.3, seed 0, not normalised), SQ8, global
D0 with replication fanout 2, a subtree per D0 child (fanout 2 at its root,
leaves <= 1024, k = 32), 12-bit HashPrune with R = 64, the `_mem.index`
image; 1,000 held-out queries searched from the build's entry point.

Bar: the GPU image equals the CPU build's (oracle/pybuild.py: the oracle's
restatement of every stage, fed the same points, sketches and D0 leaders)
byte for byte, so recall@10 of the two builds is equal (north star: within
0.002); the GPU search is checked against the oracle's search on a query
sample."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import datagen
from shear_amd import graph as G
from shear_amd import pipeline as P

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _truth(x, q, k):
    xd = torch.from_numpy(x).cuda().double()
    qd = torch.from_numpy(q).cuda().double()
    dd = (qd * qd).sum(1, keepdim=True) - 2.0 * (qd @ xd.t()) + (xd * xd).sum(1)[None, :]
    return torch.topk(dd, k, dim=1, largest=False).indices.cpu().numpy()


def _reachable(targets, counts, start):
    n = targets.shape[0]
    valid = torch.arange(targets.shape[1], device=targets.device)[None, :] < counts[:, None]
    seen = torch.zeros(n, dtype=torch.bool, device=targets.device)
    seen[start] = True
    frontier = torch.tensor([start], device=targets.device)
    while frontier.numel():
        nb = targets[frontier][valid[frontier]].long()
        nb = torch.unique(nb[~seen[nb]])
        seen[nb] = True
        frontier = nb
    return int(seen.sum().item())


def test_c1_gpu_build_equals_cpu_build(gpu, orc):
    from oracle import pybuild as PB

    x, q = datagen.c1_numpy()
    rows, dim = x.shape
    p = P.GraphBuildParams()  # fanout 2 / 2, leaves <= 1024, k 32, R 64, 12-bit hashes
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    sk = P.sketches_of(x, P.sketch_planes(dim, p.m_hash_bits, 7))
    xg = torch.from_numpy(x).to(gpu)
    built = P.build_graph(xg, torch.from_numpy(sk).to(gpu), lead, p)
    img = built.image.cpu().numpy().tobytes()
    cpu = PB.build_graph_cpu(x, sk, lead, p)
    assert built.start == cpu["start"]
    assert len(img) == len(cpu["image"]) and img == cpu["image"], "GPU and CPU graph images differ"
    counts = built.counts.cpu().numpy()
    assert counts.max() <= p.l_max and counts.min() >= 1
    # recall@10 of both builds on the same queries (identical graphs, so
    # identical searches; the GPU search is checked against the oracle's)
    truth = _truth(x, q, 10)
    ids, dist, cmps = G.greedy_search(xg, built.targets, built.counts, built.start, torch.from_numpy(q).to(gpu),
                                      64, 10)
    gpu_recall = G.recall_at_k(ids.cpu().numpy(), truth, 10)
    t = np.full((rows, p.l_max), 0xFFFFFFFF, np.uint32)
    for i, r in enumerate(cpu["rows"]):
        t[i, : len(r)] = r
    ns = 200
    wi, wd, wc = orc.greedy_search(x, t, np.array([len(r) for r in cpu["rows"]], np.uint32), cpu["start"], q[:ns],
                                   64, 10)
    gi = ids[:ns].cpu().numpy().view(np.uint32)
    assert np.array_equal(gi, wi) and np.array_equal(dist[:ns].cpu().numpy().view(np.uint32), wd.view(np.uint32))
    cpu_recall_sample = G.recall_at_k(wi, truth[:ns], 10)
    assert abs(G.recall_at_k(gi, truth[:ns], 10) - cpu_recall_sample) <= 0.002
    reach = _reachable(built.targets, built.counts, built.start)
    print(f"C1: recall@10 (L=64) {gpu_recall:.4f}, reachable from the entry point {reach} of {rows}, "
          f"GPU build {built.build_s * 1e3:.0f} ms, CPU build {cpu['build_s']:.1f} s")
