"""Checks shared by the large end-to-end build tests (C3, C4): a per-child
observer for pipeline.build_graph_sq8 that collects what the oracle can check
on samples, and the verification itself.

  * every D0 child's leaves hold <= leaf_max rows, every point lands in at
    least one leaf, and each child emits exactly sum 2 * rows * k_eff records
    (TierLift, and the device reservoirs' source-grouped segments unless the
    build leaves out the repeats of mutual pairs, when it emits that less one
    record per mutual slot); segments: one per leaf row, their counts summing
    to the records, and on sampled leaves exactly 2 * valid slots (less the
    mutual slots, found on the host, when any record was left out);
  * a few leaves of a few children equal the oracle's leaf top-k bit for bit
    (ids and f32 distance bits);
  * the reservoirs of sampled points equal the oracle's reservoirs over every
    record those points received, with the build's backfill policy if any
    (HashPrune is a reduction: its state is a function of the record set, so
    the sample is exact);
  * degrees <= R, every point has a neighbour, and the image holds every row."""
from __future__ import annotations

import numpy as np
import torch

from gpu_helpers import assert_same
from shear_amd import edges as E


class BuildObserver:
    """Called by pipeline.build_graph_sq8 once per batch of emitted records;
    ``check_calls`` are the call indices whose leaves are sampled."""

    def __init__(self, rows: int, device, check_calls=(0, 4, 8), sample_points: int = 4096, seed: int = 3):
        self.covered = torch.zeros(rows, dtype=torch.bool, device=device)
        rng = np.random.default_rng(seed)
        self.sample = torch.from_numpy(np.sort(rng.choice(rows, sample_points, replace=False))).to(device)
        self.in_sample = torch.zeros(rows, dtype=torch.bool, device=device)
        self.in_sample[self.sample] = True
        self.sampled_records = []
        self.leaf_checks = []
        self.max_leaf = 0
        self.calls = 0
        self.check_calls = set(check_calls)

    def __call__(self, tag, cg, out, lay, rec, cnt, segs=None, nseg=0):
        sizes = out.leaf_sizes[: out.leaf_count].long()
        self.max_leaf = max(self.max_leaf, int(sizes.max().item()))
        call = self.calls
        self.calls += 1
        if self.calls % 100 == 0:
            print(f"  {self.calls} record batches built", flush=True)
        local = out.leaf_row_ids[: out.leaf_rows].long()
        self.covered[local if cg is None else cg.long()[local]] = True
        kk = torch.clamp(sizes - 1, max=out.k)
        full = int((2 * sizes * kk).sum().item())
        if segs is None:
            assert int(cnt) == full, f"{tag}: record count"
        else:
            assert int(cnt) <= full, f"{tag}: record count"
            assert nseg == int(sizes.sum().item()), f"{tag}: one segment per leaf row"
            seg_counts = segs[:nseg, 3].long()
            assert int(seg_counts.sum().item()) == int(cnt), f"{tag}: segment counts"
        r = rec[:cnt]
        self.sampled_records.append(r[self.in_sample[r[:, 0].long()]].clone())
        if call in self.check_calls:
            starts = out.leaf_starts[: out.leaf_count].cpu().numpy()
            sz = sizes.cpu().numpy()
            li = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
            g = li if cg is None else cg.cpu().numpy().view(np.uint32)[li]
            li = np.arange(len(li))
            ids = out.topk_ids[: out.leaf_rows * out.k].cpu().numpy().view(np.uint32).reshape(-1, out.k)
            dd = out.topk_dists[: out.leaf_rows * out.k].cpu().numpy().reshape(-1, out.k)
            seg0 = np.concatenate([[0], np.cumsum(sz)])
            for leaf in np.linspace(0, out.leaf_count - 1, 4).astype(int):
                a, n = int(starts[leaf]), int(sz[leaf])
                self.leaf_checks.append((g[li[a:a + n]], ids[a:a + n], dd[a:a + n]))
                if segs is not None:
                    got = int(seg_counts[int(seg0[leaf]):int(seg0[leaf]) + n].sum().item())
                    if int(cnt) == full:  # every record emitted
                        assert got == _leaf_records(ids[a:a + n], dd[a:a + n], out.k), f"{tag}: leaf {leaf} records"
                    else:
                        assert got == _unique_records(g[li[a:a + n]], ids[a:a + n], dd[a:a + n], out.k), \
                            f"{tag}: leaf {leaf} records without mutual repeats"

    def verify(self, built, sq8, p, orc, leaf_max: int, what: str) -> None:
        rows = sq8.rows
        assert self.max_leaf <= leaf_max, f"{what}: leaf of {self.max_leaf} rows above {leaf_max}"
        assert bool(self.covered.all()), f"{what}: a point is in no leaf"
        assert self.leaf_checks, f"{what}: no leaf sampled"
        counts = built.counts
        assert int(counts.max().item()) <= p.l_max and int(counts.min().item()) >= 1
        assert built.image.numel() == 24 + 4 * (rows + int(counts.sum().item()))
        k = p.leaf_knn
        for gl, ids, dd in self.leaf_checks:
            gi = torch.from_numpy(gl.astype(np.int64)).to(sq8.codes.device)
            want_ids, want_d = orc.leaf_topk(sq8.codes[gi].cpu().numpy(), sq8.scales[gi].cpu().numpy(),
                                             sq8.norms[gi].cpu().numpy(), gl, np.arange(len(gl), dtype=np.uint32),
                                             [0], [len(gl)], k)
            assert_same(ids.reshape(-1), dd.reshape(-1), want_ids, want_d, f"{what} leaf sample")
        rec = E.records_to_numpy(torch.cat(self.sampled_records), sum(int(r.shape[0]) for r in self.sampled_records))
        pos = np.full(rows, -1, np.int64)
        sample_h = self.sample.cpu().numpy()
        pos[sample_h] = np.arange(len(sample_h))
        rec = rec.copy()
        rec["src"] = pos[rec["src"].astype(np.int64)].astype(np.uint32)
        bf = getattr(p, "hashprune_backfill", None)
        if bf is not None and bf.mode != "off":
            wt, _, _, wc, _ = orc.hashprune_rhalf_reduce(len(sample_h), p.l_max, rec, mode=bf.mode,
                                                         hash_quota=bf.hash_quota or 0,
                                                         row_cap=bf.max_backfill_per_row or 0,
                                                         priority_alpha=bf.soft_tier_priority_alpha or 0.0)
        else:
            wt, _, _, wc = orc.hashprune_reduce(len(sample_h), p.l_max, rec)
        gt = built.targets[self.sample].cpu().numpy().view(np.uint32)
        gc = counts[self.sample].cpu().numpy()
        assert np.array_equal(gc, wc), f"{what}: sampled reservoir sizes differ"
        for i in range(len(sample_h)):
            assert np.array_equal(gt[i, : gc[i]], wt[i, : wc[i]]), f"{what}: reservoir of point {sample_h[i]} differs"


def _leaf_records(ids, dd, k):
    """Records of one leaf: 2 per valid slot (id set, distance finite)."""
    n = ids.shape[0]
    kl = min(k, n - 1) if n > 1 else 0
    li, lb = ids[:, :kl], dd[:, :kl].view(np.uint32)
    return int(2 * ((li != 0xFFFFFFFF) & ((lb & 0x7F800000) != 0x7F800000)).sum())


def _unique_records(gl, ids, dd, k):
    """Records of one leaf with the mutual pairs' repeats left out: 2 per
    valid slot less one per slot (r -> j) whose row j lists gl[r] at the same
    distance bits."""
    n = len(gl)
    kl = min(k, n - 1) if n > 1 else 0
    if kl == 0:
        return 0
    li, lb = ids[:, :kl], dd[:, :kl].view(np.uint32)
    valid = (li != 0xFFFFFFFF) & ((lb & 0x7F800000) != 0x7F800000)
    order = np.argsort(gl, kind="stable")
    pos = order[np.searchsorted(gl, li, sorter=order).clip(0, n - 1)]
    assert np.all(~valid | (gl[pos] == li)), "a top-k id outside its leaf"
    mutual = valid & ((li[pos] == gl[:, None, None]) & (lb[pos] == lb[:, :, None])).any(axis=2)
    return int(2 * valid.sum() - mutual.sum())


# ---- graph quality that does not depend on navigation from one entry point --
#
# Recall from the single entry point mixes two things: whether each point's
# adjacency list holds its true neighbours (the build's job) and whether
# greedy search can travel between far-apart clusters from one start.  The
# two checks below measure the first without the second, against brute force
# rather than against the CPU build, so a defect shared by the GPU build and
# its CPU restatement still shows.


def brute_knn(chunks, queries: torch.Tensor, k: int, exclude=None) -> torch.Tensor:
    """Exact k nearest rows (squared L2, f64 accumulation of f32 rows) of each
    query: ``chunks`` yields (first row, f32 device rows); ``exclude`` (int64
    per query, optional) is a row each query may not return (itself).
    Returns int64 [q, k] on the device."""
    q = queries.double()
    qn = (q * q).sum(1, keepdim=True)
    best_d = best_i = None
    sub = 1 << 18  # rows per distance block (bounds the f64 temporaries)
    for c0, xchunk in chunks:
        for s0 in range(0, xchunk.shape[0], sub):
            xc = xchunk[s0:s0 + sub]
            r0 = c0 + s0
            xd = xc.double()
            dd = qn - 2.0 * (q @ xd.t()) + (xd * xd).sum(1)[None, :]
            if exclude is not None:
                rel = exclude - r0
                hit = (rel >= 0) & (rel < xc.shape[0])
                dd[hit.nonzero().squeeze(1), rel[hit]] = float("inf")
            kk = min(k, xc.shape[0])
            d, i = torch.topk(dd, kk, dim=1, largest=False)
            i = i + r0
            if best_d is not None:
                d, j = torch.topk(torch.cat([best_d, d], 1), min(k, best_d.shape[1] + kk), dim=1, largest=False)
                i = torch.gather(torch.cat([best_i, i], 1), 1, j)
            best_d, best_i = d, i
            del xd, dd
    return best_i


def knn_coverage(targets: torch.Tensor, counts: torch.Tensor, sample: torch.Tensor, truth: torch.Tensor) -> float:
    """Mean over the sampled points of (their true nearest neighbours found in
    their adjacency list) / k; ``truth`` int64 [s, k] excludes the point itself."""
    t = targets[sample].long()
    valid = torch.arange(t.shape[1], device=t.device)[None, :] < counts[sample][:, None].long()
    t = torch.where(valid, t, torch.full_like(t, -1))
    hit = (truth[:, :, None] == t[:, None, :]).any(2)
    return float(hit.double().mean().item())


def seeded_recall(search, targets: torch.Tensor, counts: torch.Tensor, queries: torch.Tensor, truth: np.ndarray,
                  k: int = 10) -> float:
    """recall@k of searches that each start at the first graph neighbour of
    the query's true nearest point (or at that point when it has none):
    ``search(start, queries)`` returns ids [q, k]; queries sharing a start
    are searched together."""
    from shear_amd import graph as G

    nn = truth[:, 0].astype(np.int64)
    first = targets[torch.from_numpy(nn).to(targets.device), 0].cpu().numpy()
    cnt = counts[torch.from_numpy(nn).to(targets.device)].cpu().numpy()
    starts = np.where(cnt > 0, first, nn).astype(np.int64)
    found = np.zeros((len(nn), k), np.int64)
    for s in np.unique(starts):
        sel = np.nonzero(starts == s)[0]
        ids = search(int(s), queries[torch.from_numpy(sel).to(queries.device)])
        found[sel] = ids.cpu().numpy()[:, :k]
    return G.recall_at_k(found, truth, k)
