"""Pins the record -> edge restatement (oracle/tessa_edges.c) with the
reference's own fixture batch and test sketches, hash invariants, the
independent numpy restatement in brute.py and the error cases."""
import numpy as np
import pytest

import brute

F32 = np.float32
MAXID = 0xFFFFFFFF


def test_sketches(n, width):
    """build_test_sketches (leaf_build.rs:2900-2908): point * 0.1 + bit, in f32."""
    p = np.arange(n, dtype=F32)[:, None]
    b = np.arange(width, dtype=F32)[None, :]
    return (p * F32(0.1) + b).astype(F32)


test_sketches.__test__ = False


def as_tuples(rec):
    return [(int(r["src"]), int(r["dst"]), int(r["hash"]), int(r["flags"]), int(np.float32(r["dist"]).view(np.uint32)))
            for r in rec]


def test_reference_fixture_batch(orc):
    # compact_topk_evidence_fixture (leaf_build.rs:3126-3137) with the default
    # m_hash_bits = 12 (params.rs:3345).  With s_p[b] = p*0.1 + b, s_c - s_p
    # has the sign of c - p on every bit, so hash(i -> j) is 0xfff when j > i
    # and 0 when j < i.
    sk = test_sketches(31, 12)
    rec = orc.flush_compact_topk_into_edges([10, 20, 30], 2, [20, 30, 30, 10, 20, MAXID],
                                            [1.0, 2.0, 1.5, 1.0, 1.5, np.inf], sk, 12)
    f = lambda x: int(F32(x).view(np.uint32))  # noqa: E731
    want = [
        (10, 20, 0xFFF, 0, f(1.0)), (20, 10, 0, 0, f(1.0)),
        (10, 30, 0xFFF, 0, f(2.0)), (30, 10, 0, 0, f(2.0)),
        (20, 30, 0xFFF, 0, f(1.5)), (30, 20, 0, 0, f(1.5)),
        (20, 10, 0, 0, f(1.0)), (10, 20, 0xFFF, 0, f(1.0)),
        (30, 20, 0, 0, f(1.5)), (20, 30, 0xFFF, 0, f(1.5)),
    ]
    assert as_tuples(rec) == want


def test_compute_hash_invariants(orc):
    rng = np.random.default_rng(3)
    for m in (1, 7, 12, 16):
        full = (1 << m) - 1
        for _ in range(50):
            a = rng.standard_normal(16).astype(F32)
            b = rng.standard_normal(16).astype(F32)
            eq = rng.random(16) < 0.2
            b[eq] = a[eq]  # equal coordinates: both directions set the bit
            hab, hba = orc.compute_hash(a, b, m), orc.compute_hash(b, a, m)
            assert hab | hba == full                # x >= 0 or -x >= 0 for finite x
            assert orc.compute_hash(a, a, m) == full  # 0 >= 0 sets every bit
            assert hab == brute.compute_hash(a, b, m)
    # a NaN coordinate clears its bit both ways
    a = np.zeros(4, F32)
    b = np.array([1, np.nan, -1, 0], F32)
    assert orc.compute_hash(a, b, 4) == 0b1001
    assert orc.compute_hash(b, a, 4) == 0b1100


def _random_batch(rng, rows, k, universe, empty_frac=0.1):
    pids = rng.choice(universe, rows, replace=False).astype(np.uint32)
    ids = pids[rng.integers(0, rows, rows * k)].astype(np.uint32)
    d = rng.random(rows * k).astype(F32)
    ids[rng.random(rows * k) < empty_frac] = MAXID
    d[rng.random(rows * k) < 0.03] = np.inf
    d[rng.random(rows * k) < 0.03] = np.nan
    return pids, ids, d


@pytest.mark.parametrize("rows,k,m", [(1, 3, 12), (5, 4, 12), (40, 8, 16), (200, 32, 12), (64, 1, 3)])
def test_matches_independent_restatement(orc, rows, k, m):
    rng = np.random.default_rng(rows * 7 + k)
    sk = rng.standard_normal((1000, 16)).astype(F32)
    sk[rng.random(sk.shape) < 0.05] = 0.0  # exact zero differences
    pids, ids, d = _random_batch(rng, rows, k, 1000)
    got = as_tuples(orc.flush_compact_topk_into_edges(pids, k, ids, d, sk, m))
    assert got == brute.flush_edges(pids, k, ids, d, sk, m)


def test_empty_batches_emit_nothing(orc):
    sk = test_sketches(4, 12)
    assert len(orc.flush_compact_topk_into_edges([], 3, [], [], sk, 12)) == 0
    assert len(orc.flush_compact_topk_into_edges([1, 2], 0, [], [], sk, 12)) == 0
    assert len(orc.flush_compact_topk_into_edges([1, 2], 1, [MAXID, MAXID], [1.0, 1.0], sk, 12)) == 0


def test_errors(orc):
    sk = test_sketches(31, 12)
    with pytest.raises(orc.EdgeError) as e:   # leaf_build.rs:1796-1801
        orc.flush_compact_topk_into_edges([10, 20], 1, [20, 5], [1.0, 1.0], sk, 12)
    assert e.value.code == -1 and e.value.point == 5
    with pytest.raises(orc.EdgeError) as e:   # no sketch row for a point
        orc.flush_compact_topk_into_edges([10, 40], 1, [40, 10], [1.0, 1.0], sk, 12)
    assert e.value.code == -3 and e.value.point == 40
    with pytest.raises(orc.EdgeError) as e:   # m_bits above 16 / width
        orc.flush_compact_topk_into_edges([10, 20], 1, [20, 10], [1.0, 1.0], sk, 13)
    assert e.value.code == -2
