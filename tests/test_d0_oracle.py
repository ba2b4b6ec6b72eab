"""Pins of the global D0 assignment oracle (oracle/tessa_d0.c): distance
order against f64 L2 of the raw vectors when gaps exceed the SQ8 error, own
leader first, ties by leader id, full orders, and the grouping into children
(shear-core/src/algorithm/pipnn/compute_backend.rs:18016-18511,
dco_sq_int8.rs:2950-2965)."""
import numpy as np
import pytest


def _case(orc, rng, rows, dim, nl, spread=10.0):
    centres = rng.standard_normal((nl, dim)).astype(np.float32) * spread
    x = (centres[rng.integers(0, nl, rows)] + rng.standard_normal((rows, dim)).astype(np.float32)).astype(np.float32)
    codes, scales, norms = orc.quantize(x)
    lcodes, lscales, lnorms = orc.quantize(centres)
    return x, centres, (codes, scales, norms), (lcodes, lscales, lnorms)


def test_order_is_l2_when_gaps_exceed_quantization(orc):
    rng = np.random.default_rng(0)
    x, centres, (c, s, n), (lc, ls, ln) = _case(orc, rng, 300, 24, 40)
    ids = rng.permutation(1000)[:40].astype(np.uint32)
    child, _, _ = orc.d0_assign(c, s, n, np.arange(300), lc, ls, ln, ids, 3)
    d = ((x[:, None, :].astype(np.float64) - centres[None].astype(np.float64)) ** 2).sum(-1)
    order = np.argsort(d, axis=1)[:, :4]
    # SQ8 moves a distance by well under 2% of |x|^2 + |l|^2 at this dim
    bound = 0.02 * ((x.astype(np.float64) ** 2).sum(1) + (centres.astype(np.float64) ** 2).sum(1).max())
    gaps = (np.take_along_axis(d, order[:, 1:], 1) - np.take_along_axis(d, order[:, :3], 1)).min(1)
    gap_ok = gaps > bound
    assert gap_ok.sum() > 60
    assert np.array_equal(child[gap_ok], order[gap_ok, :3])


def test_own_leader_first_and_full_order(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((50, 16)) * 5).astype(np.float32)
    c, s, n = orc.quantize(x)
    ids = np.arange(50, dtype=np.uint32)[::-1].copy()
    child, offs, pts = orc.d0_assign(c, s, n, np.arange(50) + 7, c, s, n, ids, 32)
    assert np.array_equal(child[:, 0], np.arange(50))
    child_all, _, _ = orc.d0_assign(c[:20], s[:20], n[:20], np.arange(20), c, s, n, ids, 32)
    assert all(len(set(r.tolist())) == 32 for r in child_all)  # distinct leaders
    with pytest.raises(ValueError):
        orc.d0_assign(c, s, n, np.arange(50), c[:4], s[:4], n[:4], ids[:4], 5)
    with pytest.raises(ValueError):
        orc.d0_assign(c, s, n, np.arange(50), c, s, n, ids, 33)


def test_ties_by_leader_id(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((30, 8)).astype(np.float32)
    c, s, n = orc.quantize(x)
    lc, ls, ln = orc.quantize(rng.standard_normal((5, 8)).astype(np.float32))
    # every leader twice: the copy with the smaller id comes first
    lc2, ls2, ln2 = np.repeat(lc, 2, 0), np.repeat(ls, 2), np.repeat(ln, 2)
    ids = np.array([9, 3, 4, 8, 0, 1, 7, 6, 5, 2], np.uint32)
    child, _, _ = orc.d0_assign(c, s, n, np.arange(30), lc2, ls2, ln2, ids, 10)
    for r in child:
        for a, b in zip(r[0::2], r[1::2]):
            assert a // 2 == b // 2 and ids[a] < ids[b]


def test_children_group_fragments_in_row_order(orc):
    rng = np.random.default_rng(3)
    _, _, (c, s, n), (lc, ls, ln) = _case(orc, rng, 500, 12, 17, spread=1.0)
    gids = rng.permutation(5000)[:500].astype(np.uint32)
    child, offs, pts = orc.d0_assign(c, s, n, gids, lc, ls, ln, np.arange(17, dtype=np.uint32), 4)
    flat = child.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(pts, np.repeat(gids, 4)[order])
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=17))]).astype(np.uint64))
