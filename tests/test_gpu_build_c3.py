"""BASELINE configs[2] (C3) end to end on one GPU: 10,000,000 x 768 unit
vectors (1,000-component mixture, sigma 0.25, 5 % uniform outliers, seed 2;
inner product run as L2 on unit vectors), SQ8 resident in HBM, global D0 with
replication fanout 2, a subtree per D0 child (fanout 2 at its root, leaves
<= 2048, k = 32), edge records, HashPrune reservoirs (R = 64) and the
`_mem.index` image; 1,000 held-out queries searched from the entry point
against exact ground truth.

A CPU build of this size is out of reach, so parity is checked on samples
and through size-independent properties:
  * every D0 child's leaves hold <= leaf_max rows, every point lands in at
    least one leaf, and each child emits exactly sum 2 * rows * k_eff records;
  * a sample of leaves per sampled child equals the oracle's leaf top-k bit
    for bit (ids and f32 distance bits);
  * the reservoirs of 4,096 sampled points equal the oracle's reservoirs over
    every record those points received (HashPrune is a reduction: its state
    is a function of the record set, so the sample is exact);
  * degrees <= R and the image holds every row."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_same, require_gpu
from shear_amd import datagen
from shear_amd import edges as E
from shear_amd import graph as G
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
    p = P.GraphBuildParams(c_max=2048)
    leaf_max = max(256, p.c_max)
    sk = (x @ torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(gpu).t()).contiguous()
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    sq8 = T.quantize_sq_int8_matrix(x)

    covered = torch.zeros(rows, dtype=torch.bool, device=gpu)
    rng = np.random.default_rng(3)
    sample = torch.from_numpy(np.sort(rng.choice(rows, 4096, replace=False))).to(gpu)
    in_sample = torch.zeros(rows, dtype=torch.bool, device=gpu)
    in_sample[sample] = True
    sampled_records = []
    leaf_checks = []
    stats = {"max_leaf": 0, "children": 0}
    check_children = {0, 499, 998}

    def observe(c, cg, out, lay, rec, cnt):
        sizes = out.leaf_sizes[: out.leaf_count]
        stats["max_leaf"] = max(stats["max_leaf"], int(sizes.max().item()))
        stats["children"] += 1
        local = out.leaf_row_ids[: out.leaf_rows].long()
        covered[cg.long()[local]] = True
        kk = torch.clamp(sizes - 1, max=out.k)
        assert int(cnt) == int((2 * sizes * kk).sum().item()), f"child {c}: record count"
        r = rec[:cnt]
        src = r[:, 0].long()
        sampled_records.append(r[in_sample[src]].clone())
        if c in check_children:
            # up to four leaves of this child against the oracle
            starts = out.leaf_starts[: out.leaf_count].cpu().numpy()
            sz = sizes.cpu().numpy()
            g = cg.cpu().numpy().view(np.uint32)
            li = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
            ids = out.topk_ids[: out.leaf_rows * out.k].cpu().numpy().view(np.uint32).reshape(-1, out.k)
            dd = out.topk_dists[: out.leaf_rows * out.k].cpu().numpy().reshape(-1, out.k)
            for leaf in np.linspace(0, out.leaf_count - 1, 4).astype(int):
                a, n = int(starts[leaf]), int(sz[leaf])
                gl = g[li[a:a + n]]
                leaf_checks.append((gl, ids[a:a + n], dd[a:a + n]))

    built = P.build_graph_sq8(sq8, sk, lead, p, observer=observe)
    assert stats["max_leaf"] <= leaf_max
    assert bool(covered.all()), "a point is in no leaf"
    counts = built.counts
    assert int(counts.max().item()) <= p.l_max and int(counts.min().item()) >= 1
    assert built.image.numel() == 24 + 4 * (rows + int(counts.sum().item()))

    # sampled leaves against the oracle (SQ8 of the leaf's rows from the same payload)
    k = p.leaf_knn
    for gl, ids, dd in leaf_checks:
        gi = torch.from_numpy(gl.astype(np.int64)).to(gpu)
        codes = sq8.codes[gi].cpu().numpy()
        sc = sq8.scales[gi].cpu().numpy()
        nm = sq8.norms[gi].cpu().numpy()
        want_ids, want_d = orc.leaf_topk(codes, sc, nm, gl, np.arange(len(gl), dtype=np.uint32), [0], [len(gl)], k)
        assert_same(ids.reshape(-1), dd.reshape(-1), want_ids, want_d, "C3 leaf sample")

    # sampled reservoirs against the oracle over every record the points received
    rec = E.records_to_numpy(torch.cat(sampled_records), sum(int(r.shape[0]) for r in sampled_records))
    pos = np.full(rows, -1, np.int64)
    sample_h = sample.cpu().numpy()
    pos[sample_h] = np.arange(len(sample_h))
    rec = rec.copy()
    rec["src"] = pos[rec["src"].astype(np.int64)].astype(np.uint32)
    wt, _, _, wc = orc.hashprune_reduce(len(sample_h), p.l_max, rec)
    gt = built.targets[sample].cpu().numpy().view(np.uint32)
    gc = counts[sample].cpu().numpy()
    assert np.array_equal(gc, wc), "sampled reservoir sizes differ"
    for i in range(len(sample_h)):
        assert np.array_equal(gt[i, : gc[i]], wt[i, : wc[i]]), f"reservoir of point {sample_h[i]} differs"

    q = spec.queries(1000, 11, gpu)
    truth = _truth(x, q)
    res = []
    for L in (64, 256):
        ids, _, _ = G.greedy_search(x, built.targets, built.counts, built.start, q, L, 10)
        res.append((L, G.recall_at_k(ids.cpu().numpy(), truth, 10)))
    print(f"C3: build {built.build_s:.2f} s ({rows / built.build_s:,.0f} points/s), {built.stages}, recall@10 "
          + ", ".join(f"L={L}: {r:.4f}" for L, r in res))
