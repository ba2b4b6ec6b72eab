"""BASELINE configs[0] (C1) end to end: 200,000 x 128 mixture points (64
components, centres N(0, I), sigma 0.3, seed 0, not normalised), SQ8, global
D0 with replication fanout 2, a subtree per D0 child (fanout 2 at its root,
leaves <= 1024, k = 32), 12-bit HashPrune with R = 64, the `_mem.index`
image; 1,000 held-out queries searched from the build's entry point.

Bar: the GPU image equals the CPU build's (oracle/pybuild.py: the oracle's
restatement of every stage, fed the same points, sketches and D0 leaders)
byte for byte, so recall@10 of the two builds is equal (north star: within
0.002); the GPU search is checked against the oracle's search on a query
sample.

Graph quality without the single-entry navigation (against brute force, not
the CPU build, so a defect both builds share still shows): the adjacency
lists of 2,000 sampled points hold at least 60 % of their 10 true nearest
neighbours (measured 0.685), and searches started at the first graph
neighbour of each query's true nearest point reach recall@10 >= 0.9 at
L = 64 (measured 0.978).  From the entry point the same searches reach
about 0.12: the clusters lie far apart and greedy search from one start
rarely crosses between them.

The final RobustPrune (build_shear_index --final-prune) is checked the same
way: the GPU build with it equals the CPU build's table pruned by the
oracle's RobustPrune, byte for byte."""
import numpy as np
import pytest
import torch

from build_checks import brute_knn, knn_coverage, seeded_recall
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


@pytest.fixture(scope="module")
def c1(gpu):
    from oracle import pybuild as PB

    x, q = datagen.c1_numpy()
    rows, dim = x.shape
    p = P.GraphBuildParams()  # fanout 2 / 2, leaves <= 1024, k 32, R 64, 12-bit hashes
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    sk = P.sketches_of(x, P.sketch_planes(dim, p.m_hash_bits, 7))
    xg = torch.from_numpy(x).to(gpu)
    built = P.build_graph(xg, torch.from_numpy(sk).to(gpu), lead, p)
    cpu = PB.build_graph_cpu(x, sk, lead, p)
    return dict(x=x, q=q, p=p, lead=lead, sk=sk, xg=xg, built=built, cpu=cpu)


def test_c1_gpu_build_equals_cpu_build(gpu, orc, c1):
    x, q, p, xg, built, cpu = c1["x"], c1["q"], c1["p"], c1["xg"], c1["built"], c1["cpu"]
    rows = x.shape[0]
    img = built.image.cpu().numpy().tobytes()
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


def test_c1_graph_local_quality(gpu, c1):
    """Adjacency lists against brute-force neighbours, and searches seeded
    next to each query (no single-entry navigation)."""
    x, q, p, xg, built = c1["x"], c1["q"], c1["p"], c1["xg"], c1["built"]
    rows = x.shape[0]
    sample = torch.from_numpy(np.sort(np.random.default_rng(11).choice(rows, 2000, replace=False))).to(gpu)
    truth_b = brute_knn([(0, xg)], xg[sample], 10, exclude=sample)
    cov = knn_coverage(built.targets, built.counts, sample, truth_b)
    qg = torch.from_numpy(q).to(gpu)
    truth_q = brute_knn([(0, xg)], qg, 10).cpu().numpy()
    seeded = seeded_recall(lambda s, qq: G.greedy_search(xg, built.targets, built.counts, s, qq, 64, 10)[0],
                           built.targets, built.counts, qg, truth_q)
    ids, _, _ = G.greedy_search(xg, built.targets, built.counts, built.start, qg, 64, 10)
    entry = G.recall_at_k(ids.cpu().numpy(), truth_q, 10)
    print(f"C1 graph quality: 10-NN coverage of adjacency lists {cov:.4f}, recall@10 (L=64) seeded next to "
          f"the query {seeded:.4f}, from the entry point {entry:.4f}", flush=True)
    assert cov >= 0.60, f"adjacency lists hold {cov:.3f} of the true 10-NN"
    assert seeded >= 0.90, f"seeded recall@10 {seeded:.3f}"


def test_c1_final_prune_equals_cpu(gpu, orc, c1):
    """build_shear_index --final-prune: RobustPrune of every row over the f32
    points (alpha 1.2, max occlusion 750, saturate on) after HashPrune."""
    from dataclasses import replace

    x, q, p, xg, cpu = c1["x"], c1["q"], c1["p"], c1["xg"], c1["cpu"]
    rows = x.shape[0]
    pp = replace(p, final_prune=True)
    built = P.build_graph(xg, torch.from_numpy(c1["sk"]).to(gpu), c1["lead"], pp)
    t = np.full((rows, p.l_max), 0xFFFFFFFF, np.uint32)
    for i, r in enumerate(cpu["rows"]):
        t[i, : len(r)] = r
    cnt = np.array([len(r) for r in cpu["rows"]], np.uint32)
    wt, wc = orc.robust_prune(x, t, cnt, pp.l_max, pp.prune_max_occlusion, pp.prune_alpha, pp.prune_saturate)
    want = orc.graph_bytes(cpu["start"], 0, [wt[i, : wc[i]] for i in range(rows)])
    img = built.image.cpu().numpy().tobytes()
    assert built.start == cpu["start"]
    assert img == want, "GPU final-prune image differs from the CPU build pruned by the oracle"
    qg = torch.from_numpy(q).to(gpu)
    truth = brute_knn([(0, xg)], qg, 10).cpu().numpy()
    ids, _, _ = G.greedy_search(xg, built.targets, built.counts, built.start, qg, 64, 10)
    print(f"C1 with final prune: recall@10 (L=64) {G.recall_at_k(ids.cpu().numpy(), truth, 10):.4f}, mean degree "
          f"{float(built.counts.float().mean()):.1f} (without: {float(c1['built'].counts.float().mean()):.1f}), "
          f"prune {built.stages['final_prune_ms']:.1f} ms", flush=True)


def test_c1_production_backfill_equals_cpu(gpu, orc, c1):
    """build_shear_index's default HashPrune policy (SoftTier-Q3, alpha 1.02,
    at most 3 backups per underfull row, main.rs:2360-2374): the GPU image
    equals the CPU build's with the same policy, byte for byte."""
    from dataclasses import replace

    from oracle import pybuild as PB
    from shear_amd import hashprune as H

    x, q, p, xg = c1["x"], c1["q"], c1["p"], c1["xg"]
    pp = replace(p, hashprune_backfill=H.PRODUCTION_BACKFILL)
    built = P.build_graph(xg, torch.from_numpy(c1["sk"]).to(gpu), c1["lead"], pp)
    cpu = PB.build_graph_cpu(x, c1["sk"], c1["lead"], pp)
    img = built.image.cpu().numpy().tobytes()
    assert built.start == cpu["start"]
    assert img == cpu["image"], "GPU and CPU images differ with the production backfill"
    base = c1["built"].counts.cpu().numpy()
    cnt = built.counts.cpu().numpy()
    under = base < p.l_max
    assert np.all(cnt >= base) and np.all(cnt - base <= 3) and np.all(cnt[~under] == base[~under])
    qg = torch.from_numpy(q).to(gpu)
    truth = brute_knn([(0, xg)], qg, 10).cpu().numpy()
    rec = {}
    for name, b in (("with", built), ("without", c1["built"])):
        ids, _, _ = G.greedy_search(xg, b.targets, b.counts, b.start, qg, 64, 10)
        rec[name] = G.recall_at_k(ids.cpu().numpy(), truth, 10)
    print(f"C1 with the production backfill: {int((cnt > base).sum())} of {int(under.sum())} underfull rows "
          f"took {int((cnt - base).sum())} backups; recall@10 (L=64) {rec['with']:.4f} (without: "
          f"{rec['without']:.4f})", flush=True)
