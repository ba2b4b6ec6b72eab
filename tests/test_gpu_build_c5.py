"""BASELINE configs[4] (C5) end to end on one GPU: 150,000,000 x 768 unit
vectors from a 16,000-component mixture (sigma uniform in [0.15, 0.4] per
component, seed 4), generated, quantized and sketched 1,048,576 rows at a
time (the 460 GB f32 set is never resident); the SQ8 set (115 GB) and every
point's HashPrune reservoir (R = 64: 96 GB) in HBM; global D0 with
replication fanout 2, a subtree per D0 child (fanout 2 at its root, leaves
<= 1,024, k = 32), edge records, the `_mem.index` image.

The configuration asks for a 64 GB host budget with source-range spill to
NVMe; this build keeps the reservoirs in HBM instead (the 614 GB of records
would need about 550 GB of spill space, and the GPU boxes have about 80 GB of
free disk), so TierLift is not on this path.

A CPU build of this size is out of reach, so parity is checked on samples and
through size-independent properties (build_checks.BuildObserver): every leaf
within leaf_max, every point in a leaf, each D0 child's record count equal
to sum 2 * rows * k_eff, sampled leaves equal to the oracle's leaf top-k bit
for bit, 4,096 sampled reservoirs equal to the oracle's reservoirs over every
record they received, degrees <= R and the image size.  Graph quality is
measured against exact ground truth over the regenerated f32 chunks:
recall@10 of 1,000 held-out queries searched from the entry point over the
SQ8 rows, and, without single-entry navigation, the 10-NN coverage of 512
sampled points' adjacency lists and the recall of searches seeded at the
first graph neighbour of each query's true nearest point."""
import time

import numpy as np
import pytest
import torch

from build_checks import BuildObserver, brute_knn, knn_coverage, seeded_recall
from gpu_helpers import require_gpu
from shear_amd import datagen
from shear_amd import graph as G
from shear_amd import pipeline as P

pytestmark = pytest.mark.gpu

ROWS = 150_000_000


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def test_c5_build(gpu, orc):
    spec = datagen.c5_spec(ROWS)
    dim = spec.dim
    p = P.GraphBuildParams()  # fanout 2 / 2, leaves <= 1024, k 32, R 64
    leaf_max = max(256, p.c_max)
    planes = torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(gpu)
    t0 = time.perf_counter()

    def chunks():
        for i in range(spec.chunks):
            if i % 32 == 0:
                print(f"C5: chunk {i}/{spec.chunks}", flush=True)
            yield spec.chunk(i, gpu)

    sq8, sk = P.sq8_from_chunks(chunks(), ROWS, dim, planes)
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0
    torch.cuda.empty_cache()
    lead = P.d0_leader_rows(ROWS, P.d0_leader_count(ROWS, dim, p), p.random_seed)
    obs = BuildObserver(ROWS, gpu, check_calls=(0, 40, 80, 120))
    print(f"C5: {ROWS} rows generated, quantized and sketched in {gen_s:.1f} s; building", flush=True)
    built = P.build_graph_sq8(sq8, sk, lead, p, observer=obs)
    del sk
    torch.cuda.empty_cache()
    print(f"C5: build {built.build_s:.2f} s ({ROWS / built.build_s:,.0f} points/s), {built.stages}", flush=True)
    obs.verify(built, sq8, p, orc, leaf_max, "C5")
    print("C5: leaf, record-count and reservoir samples match the oracle", flush=True)

    # exact ground truth over the regenerated f32 chunks, for the queries and
    # for 512 sampled points of chunk 0 (their own row excluded)
    q = spec.queries(1000, 11, gpu)
    base = torch.from_numpy(np.sort(np.random.default_rng(5).choice(spec.chunk_rows, 512, replace=False))).to(gpu)
    base_x = spec.chunk(0, gpu)[base]
    probe = torch.cat([q, base_x])
    excl = torch.cat([torch.full((q.shape[0],), -1, dtype=torch.int64, device=gpu), base])

    def f32_chunks():
        for i in range(spec.chunks):
            yield i * spec.chunk_rows, spec.chunk(i, gpu)

    t1 = time.perf_counter()
    truth = brute_knn(f32_chunks(), probe, 10, exclude=excl)
    truth_q = truth[: q.shape[0]].cpu().numpy()
    truth_b = truth[q.shape[0]:]
    print(f"C5: exact ground truth in {time.perf_counter() - t1:.1f} s", flush=True)

    rec = {}
    for L in (64, 128, 256):
        ids, _, _ = G.greedy_search_sq8(sq8, built.targets, built.counts, built.start, q, L, 10)
        rec[L] = G.recall_at_k(ids.cpu().numpy(), truth_q, 10)
    cov = knn_coverage(built.targets, built.counts, base, truth_b)
    ns = 300
    seeded = seeded_recall(lambda s, qq: G.greedy_search_sq8(sq8, built.targets, built.counts, s, qq, 64, 10)[0],
                           built.targets, built.counts, q[:ns], truth_q[:ns])
    print(f"C5: recall@10 from the entry point L=64/128/256: {rec[64]:.4f} / {rec[128]:.4f} / {rec[256]:.4f}; "
          f"10-NN coverage of adjacency lists {cov:.4f}; recall@10 (L=64) seeded next to the query {seeded:.4f}",
          flush=True)
    # measured 0.293 and 0.822: a point's true neighbours lie in its own
    # cluster of ~9,400 points, split over ten or more leaves of <= 1,024
    assert cov >= 0.25, f"adjacency lists hold {cov:.3f} of the true 10-NN"
    assert seeded >= 0.72, f"seeded recall@10 {seeded:.3f}"
