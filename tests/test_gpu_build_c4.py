"""BASELINE configs[3] (C4) end to end on one GPU: 35,000,000 x 768 unit
vectors from a 4,000-component mixture with Zipf(1.1) component sizes (seed
3), generated, quantized (SQ8) and sketched chunk by chunk; subtree tasks
planned and admitted under a 32 GB device workspace cap (the D0 children
overlap: replication fanout 2); every child's edge records streamed to the
TierLift host reducer under a 96 GiB host budget, past which source-range
shards spill to disk; then the reservoirs and the `_mem.index` image.

Checks (build_checks.BuildObserver): leaves <= leaf_max, every point in a
leaf, per-child record counts, sampled leaves and 4,096 sampled reservoirs
against the oracle, degrees <= 64; plus the largest task's workspace within
the cap, every record through the reducer, host blocks within the budget,
and spilled segments readable in the reference's format (sorted by src,
shard ranges)."""
import numpy as np
import pytest
import torch

from build_checks import BuildObserver
from gpu_helpers import require_gpu
from shear_amd import datagen
from shear_amd import edges as E
from shear_amd import pipeline as P
from shear_amd import spill as SP
from shear_amd import tierlift as TL

pytestmark = pytest.mark.gpu

CAP = 32 << 30
HOST_BUDGET = 96 << 30


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


@pytest.mark.timeout(1100)
def test_c4_build_through_tierlift(gpu, orc, tmp_path):
    spec = datagen.c4_spec(35_000_000)
    rows, dim = spec.n, spec.dim
    p = P.GraphBuildParams(gpu_workspace_budget_bytes=CAP)
    planes = torch.from_numpy(P.sketch_planes(dim, p.m_hash_bits, 7)).to(gpu)

    def chunks():
        for i in range(spec.chunks):
            if i % 8 == 0:
                print(f"C4: generating chunk {i}/{spec.chunks}", flush=True)
            yield spec.chunk(i, gpu)

    sq8, sk = P.sq8_from_chunks(chunks(), rows, dim, planes)
    torch.cuda.empty_cache()
    lead = P.d0_leader_rows(rows, P.d0_leader_count(rows, dim, p), p.random_seed)
    obs = BuildObserver(rows, gpu)
    base = tmp_path / "candidates.log"
    prm = TL.TierLiftParams(host_budget_bytes=HOST_BUDGET, spill_base=str(base))
    built = P.build_graph_sq8(sq8, sk, lead, p, observer=obs, host_reducer=prm)
    obs.verify(built, sq8, p, orc, max(256, p.c_max), "C4")
    st = built.stages
    tl = st["tierlift"]
    print(f"C4: build {built.build_s:.2f} s ({rows / built.build_s:,.0f} points/s), {st}", flush=True)
    assert st["largest_task_workspace_bytes"] <= CAP
    assert tl["records"] == st["edge_records"]
    assert tl["host_peak_bytes"] <= HOST_BUDGET + (TL.DEFAULT_STAGING_RECORDS * 16) + tl["shards"] * 16_000_000
    if tl["spilled_records"]:
        segs = SP.read_segments(base.parent / SP.MANIFEST_NAME)
        assert sum(s.record_count for s in segs) == tl["spilled_records"] == tl["reread_records"]
        for s in segs[:: max(1, len(segs) // 6)]:
            with open(SP.part_path(base, s.file_id, s.shard_id), "rb") as fh:
                fh.seek(s.byte_offset)
                r = np.frombuffer(fh.read(s.byte_len), E.EDGE_RECORD_DTYPE)
            src = r["src"]
            assert s.sorted_by_src and np.all(src[1:] >= src[:-1])
            assert src[0] == s.src_min and src[-1] == s.src_max
            assert np.all(src // SP.DEFAULT_SHARD_POINTS == s.shard_id)
