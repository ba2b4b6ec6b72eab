"""The CPU build chain (oracle/pybuild.py): its orchestration rules checked by
hand-derived values, and the product's host-side entry point rule against
the same cases (rbc_partition.rs:4964-4985: the first point of the largest D0
child, ties to the smaller point id; empty children skipped)."""
import numpy as np

from oracle import pybuild as PB
from shear_amd import datagen
from shear_amd import pipeline as P


def test_entry_point_rule():
    # children: [5, 9] (2 points), [] (empty), [7, 3, 1] (3 points), [2, 8, 4] (3 points, first id 2 < 7)
    offs = np.array([0, 2, 2, 5, 8])
    pts = np.array([5, 9, 7, 3, 1, 2, 8, 4], np.uint32)
    assert PB.entry_point(offs, pts) == 2
    assert P.entry_point(offs, pts) == 2
    # a single largest child wins regardless of ids
    offs = np.array([0, 1, 4])
    pts = np.array([0, 9, 8, 7], np.uint32)
    assert PB.entry_point(offs, pts) == 9 and P.entry_point(offs, pts) == 9
    # no non-empty child: 0
    assert PB.entry_point(np.array([0, 0]), np.zeros(0, np.uint32)) == 0
    assert P.entry_point(np.array([0, 0]), np.zeros(0, np.uint32)) == 0


def test_record_count_uses_per_leaf_k_eff(orc):
    # leaves of fewer than k+1 rows emit min(k, n-1) slots per row, forward and reverse
    x = datagen.gmm_numpy(3000, 16, 4, 0.3, 2)
    p = P.GraphBuildParams(c_max=256, leaf_knn=32)
    lead = P.d0_leader_rows(3000, 6, p.random_seed)
    sk = P.sketches_of(x, P.sketch_planes(16, p.m_hash_bits, 7))
    r = PB.build_graph_cpu(x, sk, lead, p)
    st = r["stages"]
    assert st["terminal_depth_retries"] == 0
    # rebuild the leaf sizes the chain saw and count 2 * n * min(k, n - 1)
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(3000, dtype=np.uint32)
    lr = np.asarray(lead, np.int64)
    _, offs, pts = orc.d0_assign(codes, scales, norms, gids, codes[lr], scales[lr], norms[lr], gids[lr], p.fanout_top)
    want = 0
    for c in range(len(offs) - 1):
        a, b = int(offs[c]), int(offs[c + 1])
        if b - a < 2:
            continue
        cg = pts[a:b].astype(np.uint32)
        seed = orc.subtree_root_seed(p.random_seed, 1, b - a, 3000, p.min_recurse_size)
        plan = PB._plan(b - a, p.leaf_knn, p.max_leaders, p.fanout_second, p.c_max)
        leaves, _ = orc.subtree_partition(codes[cg], scales[cg], norms[cg], seed=seed, root_depth=1,
                                          max_depth=p.max_depth, max_leaders=min(p.max_leaders, 128),
                                          fanout_second=p.fanout_second, leaf_min=plan.leaf_min,
                                          leaf_max=plan.leaf_max, psamp_fraction=p.psamp_fraction,
                                          max_leaf_count=plan.max_leaf_count, max_leaf_rows=plan.max_leaf_rows)
        want += sum(2 * len(lf) * min(p.leaf_knn, len(lf) - 1) for lf in leaves)
    assert st["edge_records"] == want
    assert len(r["rows"]) == 3000 and all(len(nb) <= p.l_max for nb in r["rows"])


def test_terminal_depth_retry_is_taken_once_and_bounds_leaves(orc):
    # tight clusters under max_depth 2: children overflow at the depth limit and are re-run with
    # max_depth 1024; every leaf of the retried run respects leaf_max
    x = datagen.gmm_numpy(20000, 64, 4, 0.05, 5)
    p = P.GraphBuildParams(max_depth=2, c_max=256)
    lead = P.d0_leader_rows(20000, 8, p.random_seed)
    sk = P.sketches_of(x, P.sketch_planes(64, p.m_hash_bits, 7))
    r = PB.build_graph_cpu(x, sk, lead, p)
    assert r["stages"]["terminal_depth_retries"] > 0
    assert r["stages"]["leaf_rows"] >= 20000
