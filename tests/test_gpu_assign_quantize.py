"""GPU parity of the assignment replay and the SQ8 quantizer with the oracle,
plus the session (host-array) API and its error reporting."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_helpers import assert_same, dev_u32, require_gpu, to_dev_sq8
from golden import make_golden as G
from shear_amd import _native as N
from shear_amd import datagen
from shear_amd import tessa as T

pytestmark = pytest.mark.gpu

FIX = np.load(G.OUT)


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


# ---- quantizer -------------------------------------------------------------------

@pytest.mark.parametrize("dim,bits", [(3, 8), (37, 8), (768, 8), (1000, 8), (128, 4), (96, 6)])
def test_quantizer_matches_oracle_bits(gpu, orc, dim, bits):
    rng = np.random.default_rng(dim * 10 + bits)
    x = (rng.standard_normal((513, dim)) * rng.uniform(1e-3, 50, (513, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :] = 127.0
    x[1, : min(dim, 6)] = [2.5, -2.5, 0.5, -0.5, 1.5, -126.5][: min(dim, 6)]
    want = orc.quantize(x, bits=bits)
    got = T.quantize_sq_int8_matrix(torch.from_numpy(x).cuda(), bits=bits)
    torch.cuda.synchronize()
    assert np.array_equal(got.codes.cpu().numpy(), want[0])
    assert np.array_equal(got.scales.cpu().numpy().view(np.uint32), want[1].view(np.uint32))
    assert np.array_equal(got.norms.cpu().numpy().view(np.uint32), want[2].view(np.uint32))


def test_quantizer_half_integer_quotients(gpu, orc):
    """Quotients x / scale on and one ulp either side of half-integers, where
    the kernel's multiply-by-reciprocal path hands over to the correctly
    rounded division; plus a row whose sum of squares overflows (finite values,
    norm +inf), rows of tiny scale and a partial last block."""
    rng = np.random.default_rng(7)
    rows, dim = 301, 64
    s = rng.uniform(1e-3, 10.0, rows).astype(np.float32)
    k = rng.integers(-126, 126, (rows, dim)).astype(np.float32)
    x = ((k + np.float32(0.5)) * s[:, None]).astype(np.float32)
    x[:, 0] = np.float32(127.0) * s  # max |x| fixes the scale near s
    step = rng.integers(-1, 2, (rows, dim))
    x = np.where(step < 0, np.nextafter(x, np.float32(-np.inf)), np.where(step > 0, np.nextafter(x, np.float32(np.inf)), x))
    x = x.astype(np.float32)
    x[5] = np.float32(1e20)          # norm overflows; codes are all 127
    x[6] *= np.float32(1e-37)        # scale below the normal range: exact division only
    x[7] = np.float32(1e-45)         # denormal values
    want = orc.quantize(x)
    got = T.quantize_sq_int8_matrix(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(got.codes.cpu().numpy(), want[0])
    assert np.array_equal(got.scales.cpu().numpy().view(np.uint32), want[1].view(np.uint32))
    assert np.array_equal(got.norms.cpu().numpy().view(np.uint32), want[2].view(np.uint32))
    assert np.isinf(want[2][5])


def test_quantizer_rejects_non_finite(gpu):
    x = torch.ones((10, 20), device="cuda")
    x[7, 3] = float("nan")
    with pytest.raises(ValueError, match="row 7"):
        T.quantize_sq_int8_matrix(x)


# ---- assignment ------------------------------------------------------------------

def _assign_dev(sq8, gids, members, leaders, mo, mc, lo, lc, rh):
    lay = T.AssignLayouts.from_host(members, leaders, mo, mc, lo, lc, rh)
    ids, d, ctr = T.assignment_replay(sq8, dev_u32(gids), lay)
    torch.cuda.synchronize()
    T.raise_on_overflow(ctr, "assignment replay")
    return ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), ctr.cpu().numpy()


@pytest.mark.parametrize("case", ["a", "b"])
def test_assignment_golden(gpu, orc, case):
    x = G.inputs_a() if case == "a" else G.inputs_b()
    rows = 607 if case == "a" else 64
    codes, scales, norms = orc.quantize(x)
    sq8 = to_dev_sq8(codes, scales, norms)
    gids = np.arange(codes.shape[0], dtype=np.uint32)
    ids, d, ctr = _assign_dev(sq8, gids, np.arange(rows), np.arange(16), [0], [rows], [0], [16], [2])
    assert_same(ids, d, FIX[f"{case}_assign_ids"], FIX[f"{case}_assign_dbits"].view(np.float32), case)
    assert ctr[N.C_ASSIGN_ROWS] == rows


def test_assignment_multi_task_matches_oracle(gpu, orc):
    x = datagen.gmm_numpy(6000, 768, 16, 0.25, seed=2)
    codes, scales, norms = orc.quantize(x)
    rng = np.random.default_rng(1)
    gids = rng.permutation(1 << 22)[:6000].astype(np.uint32)
    tasks = [(2500, 128, 2), (1, 1, 1), (700, 3, 3), (1500, 64, 4), (900, 33, 2)]
    members, leaders, mo, mc, lo, lc, rh = [], [], [], [], [], [], []
    for nm, nl, r in tasks:
        mo.append(len(members))
        mc.append(nm)
        members += rng.integers(0, 6000, nm).tolist()
        lo.append(len(leaders))
        lc.append(nl)
        leaders += rng.choice(6000, nl, replace=False).tolist()
        rh.append(r)
    sq8 = to_dev_sq8(codes, scales, norms, 768)
    ids, d, _ = _assign_dev(sq8, gids, members, leaders, mo, mc, lo, lc, rh)
    want_ids, want_d = orc.assign_replay(codes, scales, norms, gids, members, leaders, mo, mc, lo, lc, rh)
    assert_same(ids, d, want_ids, want_d, "assignment")
    # versus the CPU D0 strict order: differences only where the candidates are near-ties
    s_ids, s_d = orc.assign_strict(codes, scales, norms, gids, members, leaders, mo, mc, lo, lc, rh)
    same = ids == s_ids
    # same leader -> same f32 distance bits (well inside the 1e-5 relative bar)
    assert np.array_equal(d[same].view(np.uint32), s_d[same].view(np.uint32))
    # a different leader at a rank only where the strict order sees a near-tie
    diff = np.nonzero(~same)[0]
    assert np.all(np.abs(d[diff] - s_d[diff]) <= 2 * 2e-5)
    assert len(diff) < 0.01 * len(ids)


def test_assignment_tie_key_on_identical_leaders(gpu, orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((70, 64)).astype(np.float32)
    x[64:] = x[63]  # seven identical leaders
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(70, dtype=np.uint32) + 1000
    sq8 = to_dev_sq8(codes, scales, norms, 64)
    members, leaders = np.arange(60), np.arange(63, 70)
    ids, d, ctr = _assign_dev(sq8, gids, members, leaders, [0], [60], [0], [7], [4])
    want_ids, want_d = orc.assign_replay(codes, scales, norms, gids, members, leaders, [0], [60], [0], [7], [4])
    assert_same(ids, d, want_ids, want_d, "tie key")
    assert ctr[N.C_ASSIGN_TIE_EVENTS] > 0


# ---- session API -------------------------------------------------------------------

def _session_with(codes, scales, norms, gids):
    lib = N.load()
    h = C.c_void_p()
    N.check(lib.tessa_session_create(C.byref(N.TessaConfig(0, 0)), C.byref(h)), "create")
    view = N.Sq8View(codes.ctypes.data, scales.ctypes.data, norms.ctypes.data, gids.ctypes.data, codes.shape[0],
                     codes.shape[1], codes.shape[1])
    N.check(lib.tessa_session_upload_sq8(h, C.byref(view)), "upload")
    return lib, h


def test_session_leaf_and_assign_host_arrays(gpu, orc):
    x = datagen.gmm_numpy(3000, 128, 4, 0.3, seed=8)
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(3000, dtype=np.uint32) * 5
    lib, h = _session_with(codes, scales, norms, gids)
    try:
        members = np.arange(3000, dtype=np.uint32)
        moff = np.array([0, 1000, 2500], np.uint64)
        mcnt = np.array([1000, 1500, 500], np.uint32)
        k = 16
        ooff = np.array([0, 1000 * k, 2500 * k], np.uint64)
        ids = np.zeros(3000 * k, np.uint32)
        d = np.zeros(3000 * k, np.float32)
        ctr = np.zeros(N.COUNTER_WORDS, np.uint64)
        ms = C.c_float()
        p = lambda a: a.ctypes.data  # noqa: E731
        N.check(lib.tessa_session_leaf_topk(h, p(members), p(moff), p(mcnt), p(ooff), 3, k, N.EXEC_MFMA, p(ids),
                                            p(d), p(ctr), C.byref(ms)), "session leaf")
        want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, moff, mcnt, k)
        assert_same(ids, d, want_ids, want_d, "session leaf")
        assert ms.value > 0 and ctr[N.C_LEAF_ROWS] == 3000
        lead = np.arange(0, 3000, 50, dtype=np.uint32)
        # keep every host array alive for the duration of the call
        zero, m_cnt, l_cnt, rh = (np.array([v], np.uint32) for v in (0, 3000, len(lead), 2))
        o_off = np.array([0], np.uint64)
        aids = np.zeros(3000 * 2, np.uint32)
        ad = np.zeros(3000 * 2, np.float32)
        N.check(lib.tessa_session_assign_replay(h, p(members), p(lead), p(zero), p(m_cnt), p(zero), p(l_cnt),
                                                p(rh), p(o_off), 1, p(aids), p(ad), p(ctr), C.byref(ms)),
                "session assign")
        w_ids, w_d = orc.assign_replay(codes, scales, norms, gids, members, lead, [0], [3000], [0], [len(lead)], [2])
        assert_same(aids, ad, w_ids, w_d, "session assign")
        # invalid member ids are rejected with the reference's message tokens
        bad = members.copy()
        bad[5] = 10_000
        st = lib.tessa_session_leaf_topk(h, p(bad), p(moff), p(mcnt), p(ooff), 3, k, N.EXEC_MFMA, p(ids), p(d),
                                         p(ctr), C.byref(ms))
        assert st.code != 0 and b"overflow_flags=0x2000" in st.msg and b"INVALID_TOPK_ROW_ID" in st.msg
    finally:
        N.check(lib.tessa_session_destroy(h), "destroy")


def test_caps_report_gfx950(gpu):
    caps = N.query_caps(0)
    assert caps.arch.decode().startswith("gfx950")
    assert caps.supported == 1 and caps.compute_units >= 256
