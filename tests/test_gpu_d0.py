"""GPU parity of the global D0 assignment (tessa_global_d0_assign) with the
CPU oracle's restatement of the GPU-D0 SQ8 kernels
(shear-core/src/algorithm/pipnn/compute_backend.rs:18016-18511).
Bar: fragments, child offsets and grouped child points identical."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import _native as N
from shear_amd import d0 as D
from shear_amd import datagen
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _host(sq):
    return sq.codes.cpu().numpy(), sq.scales.cpu().numpy(), sq.norms.cpu().numpy()


def _run_case(gpu, orc, x, leader_rows, fanout, gids=None, dup=False):
    sq8 = T.quantize_sq_int8_matrix(torch.from_numpy(x).to(gpu))
    rows = sq8.rows
    gids = np.arange(rows, dtype=np.uint32) * 3 + 5 if gids is None else gids
    lr = torch.from_numpy(leader_rows).to(gpu)
    lead = T.Sq8Matrix(sq8.codes[lr].contiguous(), sq8.scales[lr].contiguous(), sq8.norms[lr].contiguous(), sq8.dim)
    lids = gids[leader_rows].copy()
    if dup:  # duplicated leaders: equal distances, the smaller id first
        lead = T.Sq8Matrix(torch.cat([lead.codes, lead.codes]), torch.cat([lead.scales, lead.scales]),
                           torch.cat([lead.norms, lead.norms]), sq8.dim)
        lids = np.concatenate([lids, lids[::-1] + 1]).astype(np.uint32)
    dg = torch.from_numpy(gids.view(np.int32)).to(gpu)
    dl = torch.from_numpy(lids.view(np.int32)).to(gpu)
    child, point, offs, pts = D.global_d0_assign(sq8, dg, lead, dl, fanout)
    torch.cuda.synchronize()
    c, s, n = _host(sq8)
    lc, ls, ln = _host(lead)
    wc, wo, wp = orc.d0_assign(c, s, n, gids, lc, ls, ln, lids, fanout)
    gc = child.cpu().numpy().view(np.uint32)
    bad = np.nonzero(np.any(gc != wc, 1))[0]
    assert len(bad) == 0, f"rows {bad[:8]} differ: got {gc[bad[0]]} want {wc[bad[0]]}"
    assert np.array_equal(point.cpu().numpy().view(np.uint32), np.repeat(gids[:, None], fanout, 1))
    assert np.array_equal(offs.cpu().numpy().view(np.uint64), wo)
    assert np.array_equal(pts.cpu().numpy().view(np.uint32), wp)


@pytest.mark.parametrize("seed,rows,dim,leaders,fanout", [
    (1, 5000, 128, 140, 10),     # C1 shape: 200k * 0.0007 leaders, fanout_top 10
    (2, 3000, 768, 300, 10),
    (3, 2000, 40, 33, 32),       # padded_dim 48; fanout = 32 of 33
    (4, 4097, 96, 1000, 3),
    (5, 700, 64, 5, 1),
    (6, 1500, 200, 64, 17),
    (7, 6000, 768, 1000, 2),     # C3 shape: fanout_top 2 (the two-slot kernel)
    (8, 3000, 128, 140, 2),
])
def test_assignment_matches_oracle(gpu, orc, seed, rows, dim, leaders, fanout):
    x = datagen.gmm_numpy(rows, dim, 12, 0.3, seed)
    lr = np.sort(np.random.default_rng(seed).permutation(rows)[:leaders]).astype(np.int64)
    _run_case(gpu, orc, x, lr, fanout)


def test_duplicate_leaders_and_clamped_distances(gpu, orc):
    x = datagen.gmm_numpy(1000, 32, 4, 0.05, 7)  # tight clusters: many distances clamp to 0
    lr = np.arange(0, 1000, 50, dtype=np.int64)
    _run_case(gpu, orc, x, lr, 8, dup=True)
    _run_case(gpu, orc, x, lr, 2, dup=True)


def test_argument_errors(gpu):
    sq8 = T.quantize_sq_int8_matrix(torch.randn(64, 32, device=gpu))
    g = torch.arange(64, dtype=torch.int32, device=gpu)
    lead = T.Sq8Matrix(sq8.codes[:4].contiguous(), sq8.scales[:4].contiguous(), sq8.norms[:4].contiguous(), 32)
    with pytest.raises(N.TessaError, match="fanout must be in 1..=min\\(32, leaders\\), got fanout=5 leaders=4"):
        D.global_d0_assign(sq8, g, lead, g[:4], 5)
    assert D.d0_leader_count(200_000) == 140 and D.d0_leader_count(50_000_000) == 1000


def test_sidecar_round_trip_of_gpu_quantized_rows(gpu, tmp_path):
    from shear_amd import sidecar as SC

    x = torch.from_numpy(datagen.gmm_numpy(3000, 100, 8, 0.3, 9)).to(gpu)
    sq8 = T.quantize_sq_int8_matrix(x)
    c, s, n = _host(sq8)
    SC.write_sidecar(tmp_path / "base", c, s, n, 100)
    h, c2, s2, n2 = SC.read_sidecar(tmp_path / "base", rows=3000, dim=100)
    back = T.Sq8Matrix(torch.from_numpy(c2).to(gpu), torch.from_numpy(s2).to(gpu), torch.from_numpy(n2).to(gpu), 100)
    assert h["padded_dim"] == sq8.padded_dim == 112
    assert torch.equal(back.codes, sq8.codes) and torch.equal(back.scales, sq8.scales) and torch.equal(back.norms, sq8.norms)
