#!/usr/bin/env python3
"""TESSA leaf-operator benchmark on one MI355X.

Workload (C2): 4,096 leaves x 1,024 points x 768-d SQ8 codes quantized from a
256-component unit-normalised Gaussian mixture (sigma 0.3, seed 1), all-pairs
int8 dot products with int32 accumulation and per-row top-32 with the
reference's tie rule; output (id, dist) candidate records.  A "step" is one
pass of the leaf operator over all 4,096 leaves with inputs resident in HBM.

Prints one JSON line.  `value` is the whole-job int8 throughput in TOPS over
the K timed steps (algorithmic ops = 2*768*sum n(n-1)); `roofline.achieved`
divides the same ops by the average duration of the dominant kernel
(leaf_mfma_kernel), measured with hipEvents recorded around it on the stream
it is launched on (tessa_leaf_topk_profiled).  `cpu_baseline` times the CPU oracle (the repo's C
restatement of the reference CPU semantics, OpenMP) on a bounded sample of
the same leaves, and the same sample is checked bit for bit against the GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

LEAVES = 4096
LEAF_ROWS = 1024
DIM = 768
K = 32
COMPONENTS = 256
SIGMA = 0.3
SEED = 1
HERE = os.path.dirname(os.path.abspath(__file__))
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--leaves", type=int, default=LEAVES)
    ap.add_argument("--cpu-budget-s", type=float, default=15.0,
                    help="approximate seconds of CPU oracle work for cpu_baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-json", default=os.path.join(HERE, "profiles", "leaf_mfma_c2_traffic.json"),
                    help="measured HBM bytes per launch of leaf_mfma_kernel (rocprofv3 --pmc FETCH_SIZE and "
                         "WRITE_SIZE, scaled by a copy kernel; see profiles/leaf_mfma_c2_traffic.md)")
    ap.add_argument("--subtree-rows", type=int, default=10_000_000,
                    help="rows of the in-HBM subtree leg (C3: 10M x 768, leaves <= 2048, fanout 2, k=32)")
    ap.add_argument("--no-subtree", action="store_true", help="skip the subtree (partition + leaf top-k) leg")
    ap.add_argument("--subtree-only", action="store_true",
                    help="run only the subtree leg and print its JSON (for profiling the partition walk)")
    ap.add_argument("--no-build", action="store_true", help="skip the C3 full-build leg")
    ap.add_argument("--build-rows", type=int, default=10_000_000,
                    help="rows of the C3 full-build leg (BASELINE configs[2]: 10,000,000)")
    ap.add_argument("--no-hashprune", action="store_true", help="skip the HashPrune reservoir leg")
    ap.add_argument("--no-recall", action="store_true", help="skip the end-to-end graph build + recall leg")
    ap.add_argument("--no-edges", action="store_true",
                    help="skip the record-emission leg (top-k slots -> SpillRecord16 edge records)")
    ap.add_argument("--c5-rows", type=int, default=0,
                    help="run only the out-of-memory build leg (BASELINE configs[4]: 150,000,000 rows as "
                         "specified) at this many rows and print its JSON line instead")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only measure the sustained int8 MFMA rate of this GPU (tessa_probe_mfma_rate) and print it")
    ap.add_argument("--no-mfma-ceiling", action="store_true",
                    help="leave the sustained int8 MFMA rate out of the default run's line")
    ap.add_argument("--copy-calibration-mib", type=str, default="",
                    help="after the timed steps, run one int32 elementwise copy kernel per size in this "
                         "comma-separated list of MiB (read N, write N) so rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE "
                         "can be scaled (two sizes cross-check the factor)")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (the TESSA operator has no multi-GPU path in this "
              f"build; see DESIGN.md for how it would shard); got --gpus {args.gpus}, WORLD_SIZE {world}",
              file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from shear_amd import _native as N
    from shear_amd import datagen
    from shear_amd import tessa as T

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    N.load()
    if args.mfma_ceiling:
        print(json.dumps(mfma_ceiling()), flush=True)
        return 0
    if args.c5_rows:
        print(json.dumps(c5_leg(dev, args.c5_rows)), flush=True)
        return 0
    if args.subtree_only:
        print(json.dumps(subtree_leg(args.subtree_rows, dev, check=False, runs=3)), flush=True)
        return 0
    leaves = args.leaves
    rows = leaves * LEAF_ROWS

    t0 = time.time()
    x = datagen.gmm_torch(rows, DIM, COMPONENTS, SIGMA, SEED, device=dev)
    sq8 = T.quantize_sq_int8_matrix(x)
    del x
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    log(f"generated + quantized {rows}x{DIM} in {time.time() - t0:.1f}s")

    gids = torch.arange(rows, dtype=torch.int32, device=dev)
    lay = T.LeafLayouts.contiguous(leaves, LEAF_ROWS, K, device=dev)
    out_ids = torch.empty(lay.output_len, dtype=torch.int32, device=dev)
    out_d = torch.empty(lay.output_len, dtype=torch.float32, device=dev)
    ctr = torch.zeros(N.COUNTER_WORDS, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream()

    phases: list = []

    def step(profiled=False):
        T.leaf_topk(sq8, gids, lay, K, executor=N.EXEC_MFMA, out_ids=out_ids, out_dists=out_d, counters=ctr,
                    stream=stream, phase_ms=phases if profiled else None)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    T.raise_on_overflow(ctr, "leaf top-k")
    log(f"warmup {args.warmup} done")

    ctr.zero_()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for i in range(args.steps):
        evs[i][0].record(stream)
        step(profiled=True)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    launch_ms = [a.elapsed_time(b) for a, b in evs]
    ph = np.array(phases, dtype=np.float64)  # [steps, 5]: MFMA filter, select, chain replay, exact re-run, batches
    T.raise_on_overflow(ctr, "leaf top-k")
    c = ctr.cpu().numpy()
    log(f"timed {args.steps} steps: wall {wall * 1e3:.2f} ms, launch median {np.median(launch_ms):.3f} ms")

    for mib in [int(v) for v in args.copy_calibration_mib.split(",") if v.strip()]:
        n = mib << 18
        src = torch.ones(n, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.add(src, 1, out=dst)  # one plain elementwise kernel: n*4 B read, n*4 B written
        torch.cuda.synchronize()
        log(f"copy calibration: {n * 4} B read, {n * 4} B written")
        del src, dst

    pairs = leaves * LEAF_ROWS * (LEAF_ROWS - 1)
    ops = 2.0 * DIM * pairs
    value_tops = ops * args.steps / wall / 1e12
    # dominant kernel: leaf_mfma_kernel (the MFMA filter), launched once per
    # batch of work items, timed with hipEvents on its stream; per launch:
    # the batch's share of the step's int8 ops over the launch's average time
    batches = int(ph[0, 4])
    ops_launch = ops / batches
    avg_kernel_s = float(np.mean(ph[:, 0])) / batches / 1e3
    achieved = ops_launch / avg_kernel_s / 1e12
    records_bytes = rows * K * 8
    survivors = float(c[N.C_LEAF_SURVIVORS]) / max(1, int(c[N.C_LEAF_ROWS]))
    # the filter's algorithmic bytes: each leaf's codes, member ids, scales and
    # norms read once; the survivor log entries (8 B each) and 16 B of row
    # metadata written per row
    algo_bytes = (rows * (DIM + 12) + rows * survivors * 8 + rows * 16) / batches

    traffic = None
    if args.traffic_json and os.path.exists(args.traffic_json) and leaves == LEAVES:
        with open(args.traffic_json) as f:
            tj = json.load(f)  # measured on this same C2 workload
        if tj.get("launches_per_step") == batches:
            traffic = tj.get("hbm_bytes_per_launch")

    result = {
        "metric": "TESSA leaf int8 TOPS (% MFMA peak)",
        "value": round(value_tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"C2 TESSA leaf microbench: {leaves} leaves x {LEAF_ROWS} pts x {DIM}-d SQ8, k={K}, "
                        f"{COMPONENTS}-comp GMM sigma={SIGMA} unit-norm, seed {SEED}",
            "leaves": leaves, "leaf_rows": LEAF_ROWS, "padded_dim": DIM, "k": K,
            "executor": "mfma (v_mfma_i32_32x32x32_i8)",
        },
        "pct_int8_mfma_peak": round(100.0 * value_tops / INT8_PEAK_TOPS, 2),
        "pair_distances_per_s": pairs * args.steps / wall,
        "records_gb_per_s": records_bytes * args.steps / wall / 1e9,
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TOPS",
            "frac": round(achieved / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "traffic_source": os.path.relpath(args.traffic_json, HERE) if traffic is not None else None,
            "kernel": "leaf_mfma_kernel",
            "launches_per_step": batches,
            "ops_per_launch": ops_launch,
            "algorithmic_hbm_bytes_per_launch": round(algo_bytes),
            "launch_ms_mean": round(float(np.mean(ph[:, 0])) / batches, 4),
            "kernel_ms_per_step_mean": round(float(np.mean(ph[:, 0])), 4),
            "kernel_ms_per_step_min": round(float(np.min(ph[:, 0])), 4),
            "kernel_ms_per_step_max": round(float(np.max(ph[:, 0])), 4),
            "select_ms_per_step_mean": round(float(np.mean(ph[:, 1])), 4),
            "chain_replay_ms_mean": round(float(np.mean(ph[:, 2])), 4),
            "exact_rerun_ms_mean": round(float(np.mean(ph[:, 3])), 4),
            "operator_ms_median": round(float(np.median(launch_ms)), 4),
        },
        "counters": {
            "rows_per_step": int(c[N.C_LEAF_ROWS]) // args.steps,
            "exact_reruns_per_step": int(c[N.C_LEAF_FALLBACK_ROWS]) // args.steps,
            "list_overflow_rows_per_step": int(c[N.C_LEAF_LIST_OVERFLOW_ROWS]) // args.steps,
            "gap_fallback_rows_per_step": int(c[N.C_LEAF_GAP_FALLBACK_ROWS]) // args.steps,
            "chain_rows_per_step": int(c[N.C_LEAF_CHAIN_ROWS]) // args.steps,
            "survivors_per_row": float(c[N.C_LEAF_SURVIVORS]) / max(1, int(c[N.C_LEAF_ROWS])),
            "final_candidates_per_row": float(c[N.C_LEAF_FINAL_CANDIDATES]) / max(1, int(c[N.C_LEAF_ROWS])),
            "refines_per_wave": float(c[N.C_LEAF_REFINES]) / max(1, int(c[N.C_LEAF_ROWS]) // 32),
        },
        "cpu_baseline": None,
    }

    if not args.no_mfma_ceiling:
        # the practical ceiling of the roofline above, measured on this GPU
        result["mfma_ceiling"] = mfma_ceiling()
        result["mfma_ceiling"]["filter_frac_of_sustained"] = round(achieved / result["mfma_ceiling"]["tops"], 4)

    if not args.no_edges:
        result["record_emission"], rec, rec_count = edge_leg(gids, lay, out_ids, out_d, stream, args.steps,
                                                             args.warmup)
        if not args.no_hashprune:
            result["hashprune"] = hashprune_leg(rec, rec_count, gids.numel(), stream, args.steps, args.warmup,
                                                check=not args.no_cpu_baseline, gids=gids, lay=lay,
                                                out_ids=out_ids, out_d=out_d)
        del rec
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        result["cpu_baseline"], result["parity_sample"] = cpu_baseline(sq8, out_ids, out_d, args.cpu_budget_s)

    if not args.no_recall:
        # BASELINE configs[0] as specified, with the CPU build beside it
        result["graph_recall"] = recall_leg(dev, check=not args.no_cpu_baseline)
        torch.cuda.empty_cache()

    if not args.no_subtree or not args.no_build:
        del out_ids, out_d, sq8, gids, lay
        torch.cuda.empty_cache()
    if not args.no_subtree:
        result["subtree"] = subtree_leg(args.subtree_rows, dev, check=not args.no_cpu_baseline)
        torch.cuda.empty_cache()
    if not args.no_build:
        result["build_c3"] = build_leg(args.build_rows, dev, check=not args.no_cpu_baseline)
        torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)
    return 0


def mfma_ceiling(workgroups=512, chains=4, seconds=0.6):
    """Sustained int8 MFMA rate of this GPU (tessa_probe_mfma_rate): random
    register operands, no memory traffic, 2 waves per SIMD with 4 chains each
    (the fastest shape measured), run long enough (about `seconds`) for the
    clock to settle under the power limit.  The leaf filter's roofline
    `peak` stays the published 5.0 POP/s; this is what the chip sustains."""
    import ctypes as C

    from shear_amd import _native as N

    lib = N.load()
    tops, mhz = C.c_double(0.0), C.c_double(0.0)
    iters = 8192
    N.check(lib.tessa_probe_mfma_rate(workgroups, chains, iters, C.byref(tops), C.byref(mhz)), "mfma probe")
    # scale the loop to the wanted duration from the short run's rate
    ops_per_iter = workgroups * 4 * chains * 65536.0
    iters = max(8192, int(seconds * tops.value * 1e12 / ops_per_iter) // 8 * 8)
    N.check(lib.tessa_probe_mfma_rate(workgroups, chains, iters, C.byref(tops), C.byref(mhz)), "mfma probe")
    log(f"sustained int8 MFMA: {tops.value:.0f} TOPS at {mhz.value:.0f} MHz "
        f"({100 * tops.value / INT8_PEAK_TOPS:.1f} % of {INT8_PEAK_TOPS:.0f})")
    return {"kernel": "v_mfma_i32_32x32x32_i8 chains on random register operands (tessa_probe_mfma_rate)",
            "workgroups": workgroups, "waves_per_simd": workgroups * 4 // 1024, "chains_per_wave": chains,
            "iterations": iters, "tops": round(tops.value, 1), "shader_mhz": round(mhz.value, 1),
            "frac_of_published_peak": round(tops.value / INT8_PEAK_TOPS, 4)}


class _LeafSampler:
    """Build observer of the bench's untimed first C3 build: keeps 4 leaves of
    each of the first `calls` record batches (point ids, top-k ids and f32
    distances) for the oracle check after the build."""

    def __init__(self, calls=3):
        self.calls, self.seen, self.leaves = calls, 0, []

    def __call__(self, tag, cg, out, lay, rec, cnt, segs=None, nseg=0):
        import numpy as np

        self.seen += 1
        if self.seen > self.calls:
            return
        lc = out.leaf_count
        starts = out.leaf_starts[:lc].cpu().numpy()
        sz = out.leaf_sizes[:lc].cpu().numpy()
        li = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
        g = li if cg is None else cg.cpu().numpy().view(np.uint32)[li]
        ids = out.topk_ids[: out.leaf_rows * out.k].cpu().numpy().view(np.uint32).reshape(-1, out.k)
        dd = out.topk_dists[: out.leaf_rows * out.k].cpu().numpy().reshape(-1, out.k)
        for leaf in np.linspace(0, lc - 1, 4).astype(int):
            a, n = int(starts[leaf]), int(sz[leaf])
            self.leaves.append((g[a:a + n].copy(), ids[a:a + n].copy(), dd[a:a + n].copy()))


def build_leg(rows, dev, check=True, nq=1000, k_recall=10, search_l=(64, 256)):
    """BASELINE configs[2] (C3) built end to end on the GPU: rows x 768 unit
    vectors (1,000 components, sigma 0.25, 5 % outliers, seed 2), SQ8, global
    D0 (fanout 2), many-root subtree runs (fanout 2, leaves <= 2048, k 32),
    source-grouped records, HashPrune (R 64) with the build_shear_index
    default policy (SoftTier-Q3 backfill, at most 3 backups per underfull
    row: BASELINE's "HashPrune cap 3"), `_mem.index`.  Two builds: the
    first (untimed for the figure: it also pays one-time set-up) samples 12
    leaves for the oracle check, the second runs with no observer and is the
    reported build time.  Recall@10 of 1,000 held-out queries against exact
    ground truth on the second build's graph."""
    import numpy as np
    import torch

    from shear_amd import datagen
    from shear_amd import graph as G
    from shear_amd import pipeline as P
    from shear_amd import tessa as T

    from shear_amd import hashprune as H

    spec = datagen.c3_spec(rows)
    x = spec.rows(dev)
    dim = x.shape[1]
    p = P.GraphBuildParams(c_max=2048, hashprune_backfill=H.PRODUCTION_BACKFILL)
    planes_t = torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(dev).t().contiguous()
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)

    def payload():
        # the build's inputs from the resident f32 rows: sketches and SQ8
        return T.quantize_sq_int8_matrix(x), (x @ planes_t).contiguous()

    sq8, sk = payload()
    torch.cuda.synchronize()
    sampler = _LeafSampler() if check else None
    first = P.build_graph_sq8(sq8, sk, lead, p, observer=sampler)
    first_s, first_image = first.build_s, first.image
    del first, sq8, sk
    torch.cuda.empty_cache()
    # the timed build starts from the f32 rows: sketching and SQ8
    # quantization are inside it
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    sq8, sk = payload()
    torch.cuda.synchronize()
    prep_s = time.perf_counter() - w0
    built = P.build_graph_sq8(sq8, sk, lead, p, t0=w0)
    same = bool(torch.equal(first_image, built.image))
    del first_image
    log(f"C3 build: {built.build_s:.3f} s ({rows / built.build_s:,.0f} points/s, sketch + SQ8 {prep_s * 1e3:.1f} ms "
        f"included; first build {first_s:.3f} s from SQ8), images identical {same}")
    res = {
        "workload": f"C3: {rows} x {dim} unit vectors (1,000 components, sigma 0.25, 5% outliers, seed 2), SQ8, "
                    f"D0 {len(lead)} leaders fanout 2, many-root subtrees fanout 2, leaves <= 2048, k 32, R 64, "
                    f"HashPrune SoftTier-Q3 cap 3",
        "build_s": round(built.build_s, 4),
        "sketch_and_sq8_ms": round(prep_s * 1e3, 2),  # inside build_s
        "first_build_s": round(first_s, 4),
        "points_per_s": round(rows / built.build_s, 1),
        "repeat_image_identical": same,
        "stages": built.stages,
        "mean_degree": round(float(built.counts.float().mean().item()), 2),
    }
    if check:
        from oracle import pyoracle as orc

        bad = slots = 0
        for gl, ids, dd in sampler.leaves:
            gi = torch.from_numpy(gl.astype(np.int64)).to(dev)
            want_ids, want_d = orc.leaf_topk(sq8.codes[gi].cpu().numpy(), sq8.scales[gi].cpu().numpy(),
                                             sq8.norms[gi].cpu().numpy(), gl, np.arange(len(gl), dtype=np.uint32),
                                             [0], [len(gl)], p.leaf_knn)
            got_i, got_d = ids.reshape(-1), dd.reshape(-1).view(np.uint32)
            bad += int(np.count_nonzero((got_i != want_ids) | (got_d != np.asarray(want_d).view(np.uint32))))
            slots += got_i.size
        res["leaf_parity_sample"] = {"leaves": len(sampler.leaves), "slots": slots, "mismatched_slots": bad}
        log(f"C3 leaf sample: {len(sampler.leaves)} leaves, {slots} slots, {bad} mismatched")
    q = spec.queries(nq, 11, dev)
    parts = []
    for s0 in range(0, rows, 1 << 20):
        xs = x[s0:s0 + (1 << 20)]
        d = (xs * xs).sum(1)[None, :] - 2.0 * (q @ xs.t())
        parts.append(torch.topk(d, 64, dim=1, largest=False).indices + s0)
    cand = torch.cat(parts, 1)
    dd = ((x[cand].double() - q.double()[:, None, :]) ** 2).sum(2)
    truth = torch.gather(cand, 1, torch.topk(dd, k_recall, dim=1, largest=False).indices).cpu().numpy()
    del cand, dd, parts
    rec = []
    for L in search_l:
        torch.cuda.synchronize()
        s0 = time.perf_counter()
        ids, _, _ = G.greedy_search(x, built.targets, built.counts, built.start, q, L, k_recall)
        torch.cuda.synchronize()
        rec.append({"L": L, "recall_at_10": round(G.recall_at_k(ids.cpu().numpy(), truth, k_recall), 4),
                    "qps": round(nq / (time.perf_counter() - s0), 1)})
    res["search"] = rec
    log(f"C3 search: {rec}")
    del x, sq8, sk, built
    return res


def c5_leg(dev, rows, nq=1000, k_recall=10, search_l=(64, 128, 256)):
    """BASELINE configs[4] (C5) on one GPU: 150,000,000 x 768 unit vectors
    from a 16,000-component mixture (sigma uniform in [0.15, 0.4], seed 4),
    generated, quantized and sketched chunk by chunk (the f32 set, 460 GB, is
    never resident); the SQ8 set (115 GB) and every point's HashPrune
    reservoir (R = 64: 96 GB) stay in HBM, D0 fanout 2, a subtree per D0
    child (fanout 2, leaves <= 1,024, k = 32), the `_mem.index` image; then
    recall@10 of 1,000 held-out queries against exact ground truth computed
    by regenerating the f32 chunks, the search reading the SQ8 rows."""
    import torch

    from shear_amd import datagen
    from shear_amd import graph as G
    from shear_amd import pipeline as P

    spec = datagen.c5_spec(rows)
    dim = spec.dim
    p = P.GraphBuildParams()
    planes = torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()

    def chunks():
        for i in range(spec.chunks):
            if i % 16 == 0:
                log(f"C5: chunk {i}/{spec.chunks}")
            yield spec.chunk(i, dev)

    sq8, sk = P.sq8_from_chunks(chunks(), rows, dim, planes)
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0
    torch.cuda.empty_cache()
    log(f"C5: {rows} rows generated, quantized and sketched in {gen_s:.1f} s")
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)

    class Progress:
        n = 0

        def __call__(self, *a):
            self.n += 1
            if self.n % 100 == 0:
                log(f"C5: {self.n} D0 children built")

    built = P.build_graph_sq8(sq8, sk, lead, p, observer=Progress())
    del sk
    torch.cuda.empty_cache()
    log(f"C5: build {built.build_s:.1f} s, {built.stages}")

    # exact ground truth: the f32 chunks regenerated, per chunk its 64 best
    # by f32 distance re-ranked in f64, then the best k over all chunks
    q = spec.queries(nq, 11, dev)
    qd = q.double()
    best_d = torch.full((nq, k_recall), float("inf"), dtype=torch.float64, device=dev)
    best_i = torch.full((nq, k_recall), -1, dtype=torch.int64, device=dev)
    t1 = time.perf_counter()
    for i in range(spec.chunks):
        x = spec.chunk(i, dev)
        d = (x * x).sum(1)[None, :] - 2.0 * (q @ x.t())
        ci = torch.topk(d, 64, dim=1, largest=False).indices
        dd = ((x[ci].double() - qd[:, None, :]) ** 2).sum(2)
        cd = torch.cat([best_d, dd], 1)
        cid = torch.cat([best_i, ci + i * spec.chunk_rows], 1)
        top = torch.topk(cd, k_recall, dim=1, largest=False).indices
        best_d, best_i = torch.gather(cd, 1, top), torch.gather(cid, 1, top)
        del x, d, ci, dd
    truth = best_i.cpu().numpy()
    truth_s = time.perf_counter() - t1
    rec = {}
    for L in search_l:
        torch.cuda.synchronize()
        s0 = time.perf_counter()
        ids, _, _ = G.greedy_search_sq8(sq8, built.targets, built.counts, built.start, q, L, k_recall)
        torch.cuda.synchronize()
        rec[f"L{L}"] = {"recall@10": round(G.recall_at_k(ids.cpu().numpy(), truth, k_recall), 4),
                        "qps": round(nq / (time.perf_counter() - s0), 1)}
    counts = built.counts
    return {
        "metric": "build points/sec (C5 out-of-memory build); graph recall@10",
        "value": round(rows / built.build_s, 1),
        "unit": "points/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"C5: {rows} x {dim} unit vectors, 16,000-component mixture, sigma U[0.15, 0.4], "
                               f"seed 4; SQ8 + reservoirs in HBM, D0 fanout 2, subtree fanout 2, leaves <= 1024, "
                               f"k 32, R 64"},
        "build_s": round(built.build_s, 2),
        "generate_quantize_sketch_s": round(gen_s, 2),
        "stages": built.stages,
        "mean_degree": round(float(counts.float().mean().item()), 2),
        "image_bytes": int(built.image.numel()),
        "truth_s": round(truth_s, 2),
        "recall": rec,
        "search": "SQ8 rows (scale * code), the f32 set is not resident",
        "peak_device_bytes": int(torch.cuda.max_memory_allocated()),
    }


def recall_leg(dev, check=True, search_l=(32, 64, 128, 256), k_recall=10, search_runs=3):
    """BASELINE configs[0] (C1) end to end on the GPU: 200,000 x 128 mixture
    points (64 components, centres N(0, I), sigma 0.3, seed 0, not
    normalised) -> shear_amd.pipeline.build_graph (SQ8, global D0 with
    replication fanout 2, a subtree per D0 child with fanout 2 at its root,
    leaves <= 1024, k = 32, 12-bit HashPrune with R = 64, `_mem.index`
    image); 1,000 held-out queries (seed 1) searched from the build's entry
    point, recall@10 against exact f64 ground truth.  With ``check`` the CPU
    build (oracle/pybuild.py, every stage restated, same inputs) is timed as
    the leg's CPU baseline and its image compared byte for byte."""
    import torch

    from shear_amd import datagen
    from shear_amd import graph as G
    from shear_amd import pipeline as P
    from shear_amd import tessa as T

    x_h, q_h = datagen.c1_numpy()
    rows, dim = x_h.shape
    p = P.GraphBuildParams()
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    sk_h = P.sketches_of(x_h, P.sketch_planes(dim, p.m_hash_bits, 7))
    x = torch.from_numpy(x_h).to(dev)
    q = torch.from_numpy(q_h).to(dev)
    sk = torch.from_numpy(sk_h).to(dev)
    # one-time library set-up (first-use kernels, workspaces) on a slice, outside the timed build
    P.build_graph(x[:8192].contiguous(), sk[:8192].contiguous(), lead[lead < 8192][:16], p)
    _ = T.quantize_sq_int8_matrix(x[:64])
    built = P.build_graph(x, sk, lead, p)
    xd, qd = x.double(), q.double()
    dd = (qd * qd).sum(1, keepdim=True) - 2.0 * (qd @ xd.t()) + (xd * xd).sum(1)[None, :]
    truth = torch.topk(dd, k_recall, dim=1, largest=False).indices.cpu().numpy()
    del xd, qd, dd
    searches = []
    for L in search_l:
        ms = []
        for _ in range(search_runs + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            ids, _, cmps = G.greedy_search(x, built.targets, built.counts, built.start, q, L, k_recall)
            b.record()
            b.synchronize()
            ms.append(a.elapsed_time(b))
        ms = ms[1:]
        searches.append({"L": L, "recall_at_10": round(G.recall_at_k(ids.cpu().numpy(), truth, k_recall), 4),
                         "qps": round(len(q_h) / (float(np.mean(ms)) / 1e3), 1),
                         "mean_distance_evals": round(float(cmps.double().mean().item()) + 1.0, 1)})
    # points reachable from the entry point (breadth-first over the rows)
    valid = torch.arange(p.l_max, device=dev)[None, :] < built.counts[:, None]
    seen = torch.zeros(rows, dtype=torch.bool, device=dev)
    seen[built.start] = True
    frontier = torch.tensor([built.start], device=dev)
    while frontier.numel():
        nb = built.targets[frontier][valid[frontier]].long()
        nb = torch.unique(nb[~seen[nb]])
        seen[nb] = True
        frontier = nb
    res = {
        "workload": f"C1: {rows} x {dim} f32 (64-comp GMM, centres N(0,I), sigma 0.3, seed 0, not normalised), SQ8, "
                    f"global D0 ({len(lead)} leaders, fanout {p.fanout_top}), a subtree per D0 child (root fanout "
                    f"{p.fanout_second}, leaves <= {p.c_max}, k={p.leaf_knn}), {p.m_hash_bits}-bit HashPrune "
                    f"R={p.l_max}; {len(q_h)} held-out queries (seed 1) from the entry point",
        "build_ms": round(built.build_s * 1e3, 2),
        "points_per_s": round(rows / built.build_s, 1),
        "stages": built.stages,
        "graph_bytes": int(built.image.numel()),
        "mean_degree": round(float(built.counts.double().mean().item()), 2),
        "max_degree": int(built.counts.max().item()),
        "start": built.start,
        "reachable_from_start": int(seen.sum().item()),
        "search": searches,
        "cpu_baseline": None,
    }
    if check:
        from oracle import pybuild as PB

        cpu = PB.build_graph_cpu(x_h, sk_h, lead, p)
        img = built.image.cpu().numpy().tobytes()
        res["cpu_baseline"] = {"value": round(rows / cpu["build_s"], 1), "unit": "points/s",
                               "cores": os.cpu_count(), "kind": "port",
                               "sample": f"the whole C1 build ({rows} points), every stage by the oracle",
                               "build_s": round(cpu["build_s"], 3), "stages": cpu["stages"],
                               "image_identical": img == cpu["image"],
                               "recall_delta": 0.0 if img == cpu["image"] else None}
    log(f"C1 build: {built.build_s * 1e3:.1f} ms, " +
        ", ".join(f"L={s_['L']} recall@10 {s_['recall_at_10']}" for s_ in searches))
    return res


def subtree_leg(rows, dev, check=True, runs=2):
    """C3-shaped resident subtree: rows x 768 unit vectors (1000-component
    mixture, sigma 0.25, 5 % uniform outliers, random order, seed 2), one
    tessa_session_run_subtree: the persistent partition walk (leaves <= 2048,
    root fanout 2, max depth 16) then the leaf top-k (k = 32) on every leaf.
    The walk's phase clocks (counter words 120, 121, 140-143: ticks of the
    100 MHz wall clock, workgroup 0's spans between grid barriers) are
    reported in ms."""
    import torch

    from shear_amd import _native as N
    from shear_amd import datagen
    from shear_amd import subtree as S
    from shear_amd import tessa as T

    t0 = time.time()
    x = datagen.c3_torch(rows, DIM, 1000, 0.25, 0.05, 2, device=dev)
    torch.cuda.synchronize()
    q0, q1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    q0.record()
    sq8 = T.quantize_sq_int8_matrix(x)
    q1.record()
    q1.synchronize()
    quantize_ms = q0.elapsed_time(q1)
    del x
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    gids = torch.arange(rows, dtype=torch.int32, device=dev)
    sess = S.SubtreeSession(0)
    sess.upload_device(sq8, gids)
    log(f"subtree: generated, quantized and uploaded {rows}x{DIM} in {time.time() - t0:.1f}s")
    # max_depth 16: one 10M-row task needs 11 levels to reach 2048-row leaves
    # (the reference's default of 10 assumes the host's D0 split first)
    params = S.PiPNNSubtreeParams(leaf_knn=K, c_max=2048, fanout_second=2, psamp_fraction=0.001, max_leaders=128,
                                  random_seed=42, max_depth=16)
    req = S.GpuSubtreePartitionRequest(point_ids=np.zeros(rows, np.uint32), parent_points=rows,
                                       min_recurse_size=64)
    out = None
    walls, part_ms, leaf_ms = [], [], []
    for i in range(runs + 1):
        out = None
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        out = sess.run(req, params)
        torch.cuda.synchronize()
        if i > 0:
            walls.append((time.perf_counter() - w0) * 1e3)
            part_ms.append(out.partition_ms)
            leaf_ms.append(out.leaf_ms)
    c = out.counters
    sizes = out.leaf_sizes[: out.leaf_count]
    pairs = int((sizes * (sizes - 1)).sum().item())
    ops = 2.0 * sq8.padded_dim * pairs
    counted_rows = int(c[N.P_LARGE_PHYSICAL_TILES]) * 16  # COUNT passes, all attempts (16-row tiles)
    assign_bytes = counted_rows * (sq8.padded_dim + 8)
    pm, lm = float(np.mean(part_ms)), float(np.mean(leaf_ms))
    res = {
        "workload": f"C3-shaped subtree: {rows} x {DIM} SQ8 (1000-comp GMM sigma 0.25, 5% outliers, unit-norm, "
                    f"seed 2), leaves <= 2048, root fanout 2, max depth 16, k={K}",
        "rows": rows,
        "leaf_rows": int(out.leaf_rows),
        "leaves": int(out.leaf_count),
        "levels": int(out.levels),
        "assignment_passes": int(c[N.P_ASSIGNMENT_PASSES]),
        "split_retries": int(c[N.P_LARGE_SPLIT_RETRIES]),
        "partition_ms": round(pm, 3),
        "partition_phase_ms": {name: round(float(c[w]) / 1e5, 3) for name, w in (
            ("walk", N.P_PARTITION_BUSY_CLOCKS), ("count", N.P_LARGE_COUNT_DISTANCE_CLOCKS),
            ("stage_plan_emit", N.P_LARGE_COUNT_COMMIT_CLOCKS), ("scatter", N.P_LARGE_SCATTER_CLOCKS),
            ("layout_and_numbering", N.P_LARGE_PUBLISH_CLOCKS), ("barrier_wait", N.P_PARTITION_WAIT_CLOCKS))},
        "partition_counted_rows": counted_rows,
        "partition_gb_per_s": round(assign_bytes / (pm / 1e3) / 1e9, 1),  # rows*(padded_dim+8) per COUNT pass
        "leaf_ms": round(lm, 3),
        "leaf_ops": ops,
        "leaf_tops": round(ops / (lm / 1e3) / 1e12, 1),
        "wall_ms": round(float(np.mean(walls)), 3),
        # SQ8 quantizer on the same rows (once, outside the runs): algorithmic
        # bytes 4*dim read + padded_dim + 8 written per row
        "quantize_ms": round(quantize_ms, 3),
        "quantize_gb_per_s": round(rows * (4 * DIM + sq8.padded_dim + 8) / (quantize_ms / 1e3) / 1e9, 1),
        "leaf_overflow_flags": int(out.leaf_counters[N.C_OVERFLOW_FLAGS]),
        "leaf_survivors_per_row": round(float(out.leaf_counters[N.C_LEAF_SURVIVORS]) / max(1, int(out.leaf_rows)), 2),
        "leaf_chain_rows": int(out.leaf_counters[N.C_LEAF_CHAIN_ROWS]),
        "leaf_exact_reruns": int(out.leaf_counters[N.C_LEAF_FALLBACK_ROWS]),
    }
    log(f"subtree: {res['leaves']} leaves, {res['leaf_rows']} rows, partition {pm:.1f} ms, leaf {lm:.1f} ms")
    if check:
        res["parity_sample"] = subtree_parity(sq8, gids, out)
    return res


def subtree_parity(sq8, gids, out, leaves=64):
    """Oracle top-k of a sample of the subtree's leaves, compared bit for bit."""
    from oracle import pyoracle as orc

    lc = out.leaf_count
    pick = np.linspace(0, lc - 1, min(leaves, lc)).astype(np.int64)
    starts = out.leaf_starts[: lc].cpu().numpy()[pick]
    sizes = out.leaf_sizes[: lc].cpu().numpy()[pick]
    rows_all = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
    members = np.concatenate([rows_all[s: s + z] for s, z in zip(starts, sizes)])
    uniq, local = np.unique(members, return_inverse=True)
    codes = sq8.codes[torch_index(uniq)].cpu().numpy()
    scales = sq8.scales[torch_index(uniq)].cpu().numpy()
    norms = sq8.norms[torch_index(uniq)].cpu().numpy()
    g = gids[torch_index(uniq)].cpu().numpy().view(np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, g, local.astype(np.uint32), offs, sizes.tolist(), out.k)
    ids = out.topk_ids.cpu().numpy().view(np.uint32)
    d = out.topk_dists.cpu().numpy()
    got_ids = np.concatenate([ids[s * out.k:(s + z) * out.k] for s, z in zip(starts, sizes)])
    got_d = np.concatenate([d[s * out.k:(s + z) * out.k] for s, z in zip(starts, sizes)])
    mism = int(np.count_nonzero((got_ids != want_ids) | (got_d.view(np.uint32) != want_d.view(np.uint32))))
    log(f"subtree parity: {len(pick)} leaves, {len(got_ids)} slots, mismatches {mism}")
    return {"leaves": int(len(pick)), "slots": int(len(got_ids)), "mismatched_slots": mism, "bit_exact": mism == 0}


def torch_index(a):
    import torch

    return torch.from_numpy(np.asarray(a, np.int64)).to("cuda:0")


def edge_leg(gids, lay, out_ids, out_d, stream, steps, warmup):
    """Record emission over the step's top-k output: every slot -> the two
    SpillRecord16 edge records of flush_compact_topk_batch_into_edges, with
    12-bit hashes from random 12-wide sketches (row = global id)."""
    import torch

    from shear_amd import edges as E

    dev = out_ids.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    sketches = torch.randn((gids.numel(), 12), generator=gen, device=dev, dtype=torch.float32)
    rec = torch.empty((2 * lay.output_len, 4), dtype=torch.int32, device=dev)
    ms = []
    count = 0
    for i in range(warmup + steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        _, count = E.emit_edge_records(gids, lay, K, out_ids, out_d, sketches, 12, out=rec, stream=stream)
        b.record(stream)
        b.synchronize()
        if i >= warmup:
            ms.append(a.elapsed_time(b))
    t = float(np.mean(ms)) / 1e3
    slots = lay.output_len
    log(f"record emission: {count} records, {np.mean(ms):.3f} ms")
    del sketches
    return {
        "kernels": "edge_count_kernel + edge_scan_kernel + edge_emit_kernel",
        "records": count,
        "ms_mean": round(float(np.mean(ms)), 4),
        "ms_min": round(float(np.min(ms)), 4),
        "slot_gb_per_s": round(slots * 8 / t / 1e9, 2),        # rows*k*8 / t
        "record_write_gb_per_s": round(count * 16 / t / 1e9, 2),
        # slots read once, records written once, one sketch row per point
        "hbm_bytes_algorithmic": slots * 8 + count * 16 + gids.numel() * 48,
        "hbm_gb_per_s_algorithmic": round((slots * 8 + count * 16 + gids.numel() * 48) / t / 1e9, 2),
        "peak_gb_per_s": HBM_PEAK_GBS,
    }, rec, count


def hashprune_leg(rec, count, num_points, stream, steps, warmup, check=True, l_max=64, sample_points=16384,
                  gids=None, lay=None, out_ids=None, out_d=None):
    """HashPrune reservoirs (l_max 64, the reference default) over the step's
    edge records, empty reservoirs each time: (a) the build's path, every
    record emitted in source-grouped order with one segment per row
    (tessa_emit_edge_segments) and merged by segments in place
    (tessa_hashprune_insert_segments); (a') the same with the repeats of
    mutual pairs left out (tessa_emit_edge_segments_unique); (b) the
    reference-order records merged by tessa_hashprune_insert (records grouped
    by source with atomics).
    The points [0, sample_points) of (a) are checked bit for bit against the
    oracle fed with all their records, and (a), (a') and (b) must be equal
    everywhere."""
    import torch

    from shear_amd import edges as E
    from shear_amd import hashprune as H

    dev = rec.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    sketches = torch.randn((gids.numel(), 12), generator=gen, device=dev, dtype=torch.float32)
    grec = torch.empty_like(rec)
    segs = torch.empty((lay.output_len // K, 4), dtype=torch.int32, device=dev)
    ms = {True: ([], []), False: ([], [])}
    ms_rec = []
    kept = {}
    with H.HashPruneReducer(num_points, l_max, dev) as hp:
        for unique in (True, False):  # the build's path last: its reservoirs are read below
            ms_emit, ms_seg = ms[unique]
            for i in range(warmup + steps):
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
                ev[0].record(stream)
                _, gcount, _, nseg = E.emit_edge_segments(gids, lay, K, out_ids, out_d, sketches, 12, out=grec,
                                                          segments=segs, stream=stream, unique=unique)
                ev[1].record(stream)
                hp.clear(stream=stream)
                hp.insert_segments(grec, segs, nseg, stream=stream)
                ev[2].record(stream)
                ev[2].synchronize()
                if i >= warmup:
                    ms_emit.append(ev[0].elapsed_time(ev[1]))
                    ms_seg.append(ev[1].elapsed_time(ev[2]))
            kept[unique] = gcount
            if unique:
                ta, hsa, da, ca = hp.slots(stream=stream)
        t, hs, d, c = hp.slots(stream=stream)
        ms_emit, ms_seg = ms[False]
        for i in range(warmup + steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            hp.clear(stream=stream)
            hp.insert(rec, count, stream=stream)  # synchronises the stream (status read-back)
            b.record(stream)
            b.synchronize()
            if i >= warmup:
                ms_rec.append(a.elapsed_time(b))
        t2, hs2, d2, c2 = hp.slots(stream=stream)
        stream.synchronize()
        same = bool(torch.equal(c, c2) and torch.equal(t, t2) and torch.equal(d, d2) and torch.equal(hs, hs2)
                    and torch.equal(c, ca) and torch.equal(t, ta) and torch.equal(d, da) and torch.equal(hs, hsa))
        filled = int((c == l_max).sum().item())
        res = {}
        if check:
            from oracle import pyoracle as orc

            r = rec[:count]
            sel = r[:, 0].view(torch.int32) < sample_points
            sub = r[sel].cpu().numpy().view(np.uint8).reshape(-1).view(orc.EDGE_DTYPE)
            wt, wh, wd, wc = orc.hashprune_reduce(sample_points, l_max, sub)
            gt = t[:sample_points].cpu().numpy().view(np.uint32)
            gh = hs[:sample_points].cpu().numpy().view(np.uint16)
            gd = d[:sample_points].cpu().numpy().view(np.uint32)
            gc = c[:sample_points].cpu().numpy().view(np.uint32)
            bad = np.nonzero((gc != wc) | np.any(gt != wt, 1) | np.any(gh != wh, 1) | np.any(gd != wd.view(np.uint32), 1))[0]
            res = {"points": sample_points, "records": int(len(sub)), "mismatched_points": int(len(bad)),
                   "bit_exact": len(bad) == 0}
        del t, hs, d, c, t2, hs2, d2, c2, ta, hsa, da, ca
    del sketches, grec, segs
    tm = float(np.mean(ms_seg)) / 1e3
    # algorithmic bytes: every record read once (16 B), every segment read
    # (16 B per row), each reservoir's slots written (10 B a slot) and its
    # count (4 B); the reservoirs start empty
    alg = gcount * 16 + nseg * 16 + num_points * (l_max * 10 + 4)
    log(f"hashprune: {count} records ({kept[True]} without mutual repeats) -> {num_points} reservoirs, segments "
        f"{np.mean(ms_seg):.3f} ms (without mutual repeats {np.mean(ms[True][1]):.3f}), records "
        f"{np.mean(ms_rec):.3f} ms, identical {same}")
    return {
        "kernels": "hp_seg_keys + radix sort + run-length encode + scan + hp_seg_gather + hp_merge_stream_kernel",
        "records": int(count),
        "records_without_mutual_repeats": int(kept[True]),
        "segments": int(nseg),
        "points": int(num_points),
        "l_max": l_max,
        "ms_mean": round(float(np.mean(ms_seg)), 4),
        "ms_min": round(float(np.min(ms_seg)), 4),
        "records_per_s": round(count / tm, 1),
        "hbm_bytes_algorithmic": int(alg),
        "hbm_gb_per_s_algorithmic": round(alg / tm / 1e9, 2),
        "peak_gb_per_s": HBM_PEAK_GBS,
        "grouped_emission_ms_mean": round(float(np.mean(ms_emit)), 4),
        "without_mutual_repeats_merge_ms_mean": round(float(np.mean(ms[True][1])), 4),
        "without_mutual_repeats_grouped_emission_ms_mean": round(float(np.mean(ms[True][0])), 4),
        "record_path_ms_mean": round(float(np.mean(ms_rec)), 4),
        "record_path_equal": same,
        "full_reservoirs": filled,
        "parity_sample": res,
    }


def cpu_baseline(sq8, out_ids, out_d, budget_s):
    """Times the CPU oracle on a bounded leaf sample and checks the GPU output on it."""
    from oracle import pyoracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    threads = max(1, min(threads, len(os.sched_getaffinity(0))))

    def run(first, count):
        r0, r1 = first * LEAF_ROWS, (first + count) * LEAF_ROWS
        codes = sq8.codes[r0:r1].cpu().numpy()
        scales = sq8.scales[r0:r1].cpu().numpy()
        norms = sq8.norms[r0:r1].cpu().numpy()
        gids = np.arange(r0, r1, dtype=np.uint32)
        members = np.arange(r1 - r0, dtype=np.uint32)
        t = time.perf_counter()
        ids, d = orc.leaf_topk(codes, scales, norms, gids, members, np.arange(count) * LEAF_ROWS,
                               [LEAF_ROWS] * count, K, threads=threads)
        return time.perf_counter() - t, ids, d

    t1, _, _ = run(0, threads)  # calibration: one leaf per thread
    count = threads * max(1, int(budget_s / max(t1, 1e-3)))
    count = min(count, sq8.rows // LEAF_ROWS)
    first = 0
    secs, ids, d = run(first, count)
    ops = 2.0 * DIM * count * LEAF_ROWS * (LEAF_ROWS - 1)
    lo, hi = first * LEAF_ROWS * K, (first + count) * LEAF_ROWS * K
    gpu_ids = out_ids[lo:hi].cpu().numpy().view(np.uint32)
    gpu_d = out_d[lo:hi].cpu().numpy()
    mism = int(np.count_nonzero((gpu_ids != ids) | (gpu_d.view(np.uint32) != d.view(np.uint32))))
    log(f"cpu oracle: {count} leaves in {secs:.2f}s on {threads} threads; GPU mismatches {mism}")
    base = {
        "value": round(ops / secs / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"{count} of {sq8.rows // LEAF_ROWS} leaves (1024 x 768, k=32), {secs:.1f}s, "
                  f"dot kernel {['scalar', 'avx2', 'avx512-vnni'][orc.dot_kernel()]}",
        "leaves_per_s": count / secs,
    }
    parity = {"leaves": count, "slots": int(hi - lo), "mismatched_slots": mism, "bit_exact": mism == 0}
    return base, parity


if __name__ == "__main__":
    sys.exit(main())
