"""BASELINE configs[2] (C3) end to end on one GPU: 10,000,000 x 768 unit
vectors (1,000-component mixture, sigma 0.25, 5 % uniform outliers, seed 2;
inner product run as L2 on unit vectors), SQ8 resident in HBM, global D0 with
replication fanout 2, a subtree per D0 child (fanout 2 at its root, leaves
<= 2048, k = 32), edge records, HashPrune reservoirs (R = 64) with the
build_shear_index default policy (SoftTier-Q3 backfill, at most 3 backups per
underfull row: "HashPrune cap 3") and the `_mem.index` image; 1,000 held-out queries searched from the entry point
against exact ground truth.

A CPU build of this size is out of reach, so parity is checked on samples
and through size-independent properties (build_checks.BuildObserver: leaf
bound, coverage, per-child record counts, sampled leaves and 4,096 sampled
reservoirs against the oracle, degrees, image size).  Graph quality without
single-entry navigation is measured against brute force: the 10-NN coverage
of 2,000 sampled points' adjacency lists and the recall of searches seeded at
the first graph neighbour of each query's true nearest point."""
import numpy as np
import pytest
import torch

from build_checks import BuildObserver, brute_knn, knn_coverage, seeded_recall
from gpu_helpers import require_gpu
from shear_amd import datagen
from shear_amd import graph as G
from shear_amd import hashprune as H
from shear_amd import pipeline as P
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _truth(x, q, k=10, chunk=1 << 20, cands=64):
    """Exact top-k: f32 candidates per chunk of rows, then f64 distances."""
    parts = []
    for s0 in range(0, x.shape[0], chunk):
        xs = x[s0:s0 + chunk]
        d = (xs * xs).sum(1)[None, :] - 2.0 * (q @ xs.t())
        parts.append(torch.topk(d, cands, dim=1, largest=False).indices + s0)
    cand = torch.cat(parts, 1)
    dd = ((x[cand].double() - q.double()[:, None, :]) ** 2).sum(2)
    return torch.gather(cand, 1, torch.topk(dd, k, dim=1, largest=False).indices).cpu().numpy()


def test_c3_build(gpu, orc):
    spec = datagen.c3_spec(10_000_000)
    x = spec.rows(gpu)
    rows, dim = x.shape
    p = P.GraphBuildParams(c_max=2048, hashprune_backfill=H.PRODUCTION_BACKFILL)
    leaf_max = max(256, p.c_max)
    sk = (x @ torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(gpu).t()).contiguous()
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    sq8 = T.quantize_sq_int8_matrix(x)

    obs = BuildObserver(rows, gpu)
    built = P.build_graph_sq8(sq8, sk, lead, p, observer=obs)
    obs.verify(built, sq8, p, orc, leaf_max, "C3")

    q = spec.queries(1000, 11, gpu)
    truth = _truth(x, q)
    res = []
    for L in (64, 256):
        ids, _, _ = G.greedy_search(x, built.targets, built.counts, built.start, q, L, 10)
        res.append((L, G.recall_at_k(ids.cpu().numpy(), truth, 10)))
    print(f"C3: build {built.build_s:.2f} s ({rows / built.build_s:,.0f} points/s), {built.stages}, recall@10 "
          + ", ".join(f"L={L}: {r:.4f}" for L, r in res), flush=True)
    sample = torch.from_numpy(np.sort(np.random.default_rng(5).choice(rows, 2000, replace=False))).to(gpu)
    cov = knn_coverage(built.targets, built.counts, sample, brute_knn([(0, x)], x[sample], 10, exclude=sample))
    ns = 300
    seeded = seeded_recall(lambda s, qq: G.greedy_search(x, built.targets, built.counts, s, qq, 64, 10)[0],
                           built.targets, built.counts, q[:ns], truth[:ns])
    print(f"C3: 10-NN coverage of adjacency lists {cov:.4f}, recall@10 (L=64) seeded next to the query "
          f"{seeded:.4f}", flush=True)
    # measured 0.426 and 0.847 (5 % of the points are uniform outliers whose
    # nearest neighbours are other outliers, rarely in the same leaf)
    assert cov >= 0.38, f"adjacency lists hold {cov:.3f} of the true 10-NN"
    assert seeded >= 0.75, f"seeded recall@10 {seeded:.3f}"
