"""The oracle reproduces the committed golden outputs for the reference's
formula-generated inputs (tests/golden/make_golden.py documents them)."""
import numpy as np
import pytest

from golden import make_golden as G

FIX = np.load(G.OUT)


@pytest.fixture(scope="module")
def case_a(orc):
    codes, scales, norms = orc.quantize(G.inputs_a())
    assert G.digest(codes, scales, norms) == str(FIX["a_digest"])
    return codes, scales, norms, np.arange(607, dtype=np.uint32)


def test_golden_digests_are_reproducible(orc):
    cb, sb, nb = orc.quantize(G.inputs_b())
    assert G.digest(cb, sb, nb) == str(FIX["b_digest"])
    assert G.digest(*G.inputs_c()) == str(FIX["c_digest"])


@pytest.mark.parametrize("k", [2, 32])
def test_oracle_matches_golden_leaf_a(orc, case_a, k):
    codes, scales, norms, gids = case_a
    ids, d = orc.leaf_topk(codes, scales, norms, gids, np.arange(607, dtype=np.uint32), [0], [607], k)
    assert np.array_equal(ids, FIX[f"a_leaf_k{k}_ids"])
    assert np.array_equal(d.view(np.uint32), FIX[f"a_leaf_k{k}_dbits"])


def test_oracle_matches_golden_leaf_c(orc):
    codes, scales, norms, gids = G.inputs_c()
    ids, d = orc.leaf_topk(codes, scales, norms, gids, np.arange(20, dtype=np.uint32), [0], [20], 4)
    assert np.array_equal(ids, FIX["c_leaf_k4_ids"])
    assert np.array_equal(d.view(np.uint32), FIX["c_leaf_k4_dbits"])
    # rows 1 and 2 are duplicates: each is the other's nearest neighbour at distance 0
    assert ids[1 * 4] == gids[2] and d[1 * 4] == 0.0
    assert ids[2 * 4] == gids[1] and d[2 * 4] == 0.0


def test_oracle_matches_golden_assignment_a(orc, case_a):
    codes, scales, norms, gids = case_a
    ids, d = orc.assign_replay(codes, scales, norms, gids, np.arange(607), np.arange(16), [0], [607], [0], [16], [2])
    assert np.array_equal(ids, FIX["a_assign_ids"])
    assert np.array_equal(d.view(np.uint32), FIX["a_assign_dbits"])
