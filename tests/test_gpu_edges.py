"""GPU parity of the candidate-record -> edge-record kernels
(tessa_emit_edge_records) with the CPU oracle's restatement of
flush_compact_topk_batch_into_edges.  Bar: every record bit-identical, in
the same order."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev_u32, require_gpu, to_dev_sq8
from shear_amd import _native as N
from shear_amd import datagen
from shear_amd import edges as E
from shear_amd import subtree as S
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu
F32 = np.float32
MAXID = 0xFFFFFFFF


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _oracle_records(orc, batches, sketches, m_bits):
    parts = [orc.flush_compact_topk_into_edges(b.point_ids, b.k, b.topk_ids, b.topk_dists, sketches, m_bits)
             for b in batches]
    return np.concatenate(parts) if parts else np.zeros(0, orc.EDGE_DTYPE)


def _same(got, want):
    assert len(got) == len(want), f"record count {len(got)} vs {len(want)}"
    g = got.view(np.uint8).reshape(-1, 16)
    w = np.ascontiguousarray(want).view(np.uint8).reshape(-1, 16)
    bad = np.nonzero(np.any(g != w, axis=1))[0]
    assert len(bad) == 0, f"{len(bad)} records differ, first at {bad[0]}: {got[bad[0]]} vs {want[bad[0]]}"


def test_reference_fixture_batch_on_gpu(gpu, orc):
    # compact_topk_evidence_fixture (leaf_build.rs:3126-3137), build_test_sketches (:2900-2908)
    sk = (np.arange(31, dtype=F32)[:, None] * F32(0.1) + np.arange(12, dtype=F32)[None, :]).astype(F32)
    b = T.CompactTopKBatch(leaf_id=17, point_ids=np.array([10, 20, 30], np.uint32), rows=3, k=2,
                           topk_ids=np.array([20, 30, 30, 10, 20, MAXID], np.uint32),
                           topk_dists=np.array([1.0, 2.0, 1.5, 1.0, 1.5, np.inf], F32))
    got = E.flush_compact_topk_batches([b], sk, 12)
    _same(got, _oracle_records(orc, [b], sk, 12))
    assert got["hash"].tolist() == [0xFFF, 0, 0xFFF, 0, 0xFFF, 0, 0, 0xFFF, 0, 0xFFF]


def _leaf_case(orc, sizes, dim, k, seed, m_bits=12, width=16):
    rng = np.random.default_rng(seed)
    n = int(sum(sizes))
    x = datagen.gmm_numpy(n, dim, 8, 0.3, seed)
    codes, scales, norms = orc.quantize(x)
    gids = rng.permutation(1 << 18)[:n].astype(np.uint32)
    # sketches are indexed by global id: a table covering every id used
    sk = np.zeros((int(gids.max()) + 1, width), F32)
    sk[gids] = rng.standard_normal((n, width)).astype(F32)
    sk[gids[: n // 7]] = np.round(sk[gids[: n // 7]])  # exact ties between coordinates
    members = rng.permutation(n).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    sq8 = to_dev_sq8(codes, scales, norms, dim)
    lay = T.LeafLayouts.from_host(members, offs, np.asarray(sizes, np.int64), k)
    g = dev_u32(gids)
    ids, d, ctr = T.leaf_topk(sq8, g, lay, k)
    torch.cuda.synchronize()
    T.raise_on_overflow(ctr, "leaf top-k")
    return gids, sk, members, offs, sizes, lay, g, ids, d


def _batches(gids, members, offs, sizes, ids, d, k):
    starts = offs.astype(np.uint64)
    return T.compact_batches_from_slices(gids, members, starts, np.asarray(sizes, np.uint64),
                                         ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), k, k)


# sketch access: rows staged in LDS for small leaves; float4 (width % 4 == 0)
# or scalar loads from HBM when a 4096-row leaf does not fit the LDS budget
@pytest.mark.parametrize("sizes,dim,k,m_bits,width", [
    ([1, 2, 3, 33, 100, 257, 1024], 48, 32, 12, 16),
    ([64] * 20 + [5, 1, 700], 32, 8, 16, 16),
    ([4096, 900], 16, 32, 12, 16),
    ([4096, 20], 16, 16, 13, 13),
    ([300, 2, 2, 41], 96, 1, 1, 16),
    ([500, 77], 24, 32, 7, 9),
])
def test_leaf_output_records_match_oracle(gpu, orc, sizes, dim, k, m_bits, width):
    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, sizes, dim, k, len(sizes) + dim, m_bits,
                                                                width)
    dsk = torch.from_numpy(sk).to(gpu)
    offsets = torch.empty(lay.leaf_count + 1, dtype=torch.int64, device=gpu)
    rec, n = E.emit_edge_records(g, lay, k, ids, d, dsk, m_bits, leaf_record_offsets=offsets)
    batches = _batches(gids, members, offs, sizes, ids, d, k)
    want = _oracle_records(orc, batches, sk, m_bits)
    _same(E.records_to_numpy(rec, n), want)
    per_leaf = np.array([2 * b.rows * b.k for b in batches], np.int64)  # every slot of a leaf top-k is valid
    assert offsets.cpu().numpy().tolist() == np.concatenate([[0], np.cumsum(per_leaf)]).tolist()


def test_empty_and_invalid_slots_are_skipped(gpu, orc):
    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, [50, 20, 9], 24, 16, 5)
    rng = np.random.default_rng(9)
    h_ids = ids.cpu().numpy().view(np.uint32).copy()
    h_d = d.cpu().numpy().copy()
    h_ids[rng.random(len(h_ids)) < 0.2] = MAXID
    h_d[rng.random(len(h_d)) < 0.05] = np.inf
    h_d[rng.random(len(h_d)) < 0.05] = np.nan
    ids2, d2 = dev_u32(h_ids), torch.from_numpy(h_d).to(gpu)
    rec, n = E.emit_edge_records(g, lay, 16, ids2, d2, torch.from_numpy(sk).to(gpu), 12)
    want = _oracle_records(orc, _batches(gids, members, offs, sizes, ids2, d2, 16), sk, 12)
    _same(E.records_to_numpy(rec, n), want)


def test_outside_leaf_id_is_rejected(gpu, orc):
    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, [40, 30, 30], 16, 8, 6)
    h_ids = ids.cpu().numpy().view(np.uint32).copy()
    # leaf 1, row 3, rank 2 gets the id of a point of leaf 0
    slot = (40 + 3) * 8 + 2
    intruder = int(gids[members[0]])
    h_ids[slot] = intruder
    h_ids[(40 + 5) * 8 + 1] = int(gids[members[1]])  # a later bad slot: not the one reported
    with pytest.raises(N.TessaError) as e:
        E.emit_edge_records(g, lay, 8, dev_u32(h_ids), d, torch.from_numpy(sk).to(gpu), 12)
    assert f"Compact top-k batch references point {intruder} outside leaf 1" in e.value.message


def test_capacity_and_sketch_errors(gpu, orc):
    gids, sk, members, offs, sizes, lay, g, ids, d = _leaf_case(orc, [30, 30], 16, 4, 7)
    dsk = torch.from_numpy(sk).to(gpu)
    small = torch.empty((10, 4), dtype=torch.int32, device=gpu)
    with pytest.raises(N.TessaError, match="capacity 10 below the 480 records needed"):
        E.emit_edge_records(g, lay, 4, ids, d, dsk, 12, out=small)
    short = dsk[: int(gids.max())].contiguous()  # the largest id loses its sketch row
    with pytest.raises(N.TessaError, match="has no sketch row"):
        E.emit_edge_records(g, lay, 4, ids, d, short, 12)


def test_subtree_output_records(gpu, orc):
    n, dim = 3000, 32
    x = datagen.gmm_numpy(n, dim, 6, 0.3, 44)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(44).permutation(1 << 16)[:n].astype(np.uint32)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    params = S.PiPNNSubtreeParams(leaf_knn=16, c_max=256, psamp_fraction=0.01, fanout_second=2, random_seed=3)
    out = sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=3 * n), params)
    torch.cuda.synchronize()
    sk = np.random.default_rng(1).standard_normal((1 << 16, 12)).astype(F32)
    lay = T.LeafLayouts(out.leaf_row_ids[: out.leaf_rows], out.leaf_starts[: out.leaf_count].to(torch.int64),
                        out.leaf_sizes[: out.leaf_count].to(torch.int32),
                        (out.leaf_starts[: out.leaf_count] * out.k).to(torch.int64),
                        int(out.leaf_sizes[: out.leaf_count].max().item()), out.leaf_rows * out.k)
    rec, cnt = E.emit_edge_records(dev_u32(gids), lay, out.k, out.topk_ids, out.topk_dists,
                                   torch.from_numpy(sk).to(gpu), 12)
    batches = T.compact_batches_from_slices(gids, out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32),
                                            out.leaf_starts[: out.leaf_count].cpu().numpy(),
                                            out.leaf_sizes[: out.leaf_count].cpu().numpy(),
                                            out.topk_ids[: out.leaf_rows * out.k].cpu().numpy().view(np.uint32),
                                            out.topk_dists[: out.leaf_rows * out.k].cpu().numpy(), out.k, 16)
    _same(E.records_to_numpy(rec, cnt), _oracle_records(orc, batches, sk, 12))
