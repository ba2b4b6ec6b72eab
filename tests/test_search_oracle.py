"""Pins of the greedy-search oracle (oracle/tessa_search.c), the recall
harness's reference: brute force on complete graphs, and hand-worked runs of
the neighbour-queue rules (shear-core/src/model/neighbor/
neighbor_priority_queue.rs:50-85; algorithm/search/search.rs:137-233)."""
import numpy as np
import pytest

from shear_amd import graph as G


def complete_graph(n):
    return np.array([[j for j in range(n) if j != i] for i in range(n)], np.uint32), np.full(n, n - 1, np.uint32)


def brute_force(x, q, k):
    """Exact top-k by squared L2 with ties by id, distances summed in
    coordinate order in f32 (the oracle's stated order)."""
    d = np.zeros((len(q), len(x)), np.float32)
    for i in range(x.shape[1]):
        t = (x[None, :, i] - q[:, None, i]).astype(np.float32)
        d = (d + (t * t).astype(np.float32)).astype(np.float32)
    idx = np.lexsort((np.broadcast_to(np.arange(len(x)), d.shape), d), axis=1)[:, :k]
    return idx.astype(np.uint32), np.take_along_axis(d, idx, 1)


@pytest.mark.parametrize("n,dim,L,K,start", [(60, 8, 64, 10, 0), (33, 5, 40, 33, 7), (100, 16, 100, 1, 99)])
def test_complete_graph_is_brute_force(orc, n, dim, L, K, start):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((12, dim)).astype(np.float32)
    t, c = complete_graph(n)
    ids, d, cmps = orc.greedy_search(x, t, c, start, q, L, K)
    want_ids, want_d = brute_force(x, q, K)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(d.view(np.uint32), want_d.view(np.uint32))
    assert np.all(cmps == n - 1)  # every point but the start scored once


def test_ties_order_by_id(orc):
    x = np.zeros((9, 3), np.float32)
    x[4] = 1.0
    t, c = complete_graph(9)
    ids, d, _ = orc.greedy_search(x, t, c, 5, np.zeros((1, 3), np.float32), 16, 9)
    assert ids[0].tolist() == [0, 1, 2, 3, 5, 6, 7, 8, 4]
    assert d[0].tolist() == [0.0] * 8 + [3.0]


def _line_graph():
    # points on a line, query at 0: dist = x^2
    x = np.array([[10], [5], [1], [3], [7], [2], [20]], np.float32)
    rows = {0: [4, 1], 1: [2, 5], 2: [6], 3: [], 4: [3], 5: [], 6: []}
    t = np.full((7, 2), 0xFFFFFFFF, np.uint32)
    c = np.zeros(7, np.uint32)
    for p, r in rows.items():
        t[p, :len(r)] = r
        c[p] = len(r)
    return x, t, c


def test_full_list_evicts_and_rejects(orc):
    # L=3 worked by hand: expand 0 -> list (25,1) (49,4) (100,0*); expand 1 ->
    # (1,2) and (4,5) go in front, evicting 0 and then 4, so 4's neighbour 3
    # (dist 9, better than 1) is never reached; expand 2 -> (400,6) is
    # rejected by the full list; 5 has no neighbours.
    x, t, c = _line_graph()
    ids, d, cmps = orc.greedy_search(x, t, c, 0, np.zeros((1, 1), np.float32), 3, 3)
    assert ids[0].tolist() == [2, 5, 1]
    assert d[0].tolist() == [1.0, 4.0, 25.0]
    assert cmps[0] == 5
    # a list long enough to keep 4 reaches 3
    ids, d, cmps = orc.greedy_search(x, t, c, 0, np.zeros((1, 1), np.float32), 5, 5)
    assert ids[0].tolist() == [2, 5, 3, 1, 4]
    assert cmps[0] == 6


def test_cursor_rewinds_to_an_insert_in_front(orc):
    # start 6 (dist 400) -> its only neighbour 0 (100) is inserted in front of
    # the cursor, which rewinds to it (without the rewind the search would end
    # there); then 0 -> 4, 1; 1 -> 2, 5 evict 0 and 6; 2's neighbour 6 is the
    # visited start; 4 (still listed) -> 3 (dist 9) evicts nothing but 4
    x, t, c = _line_graph()
    t[6, 0] = 0
    c[6] = 1
    ids, _, _ = orc.greedy_search(x, t, c, 6, np.zeros((1, 1), np.float32), 4, 4)
    assert ids[0].tolist() == [2, 5, 3, 1]


def test_short_list_pads_and_ignores_out_of_range(orc):
    x, t, c = _line_graph()
    t[3] = [0, 1000]  # out-of-range ids are skipped
    c[3] = 2
    ids, d, cmps = orc.greedy_search(x, t, c, 3, np.zeros((1, 1), np.float32), 8, 8)
    assert ids[0].tolist() == [2, 5, 3, 1, 4, 0, 6, 0xFFFFFFFF]
    with pytest.raises(ValueError):
        orc.greedy_search(x, t, c, 7, np.zeros((1, 1), np.float32), 8, 8)


def test_recall_at_k():
    found = np.array([[1, 2, 3], [4, 5, 6]])
    truth = np.array([[3, 2, 9, 1], [7, 8, 9, 4]])
    assert G.recall_at_k(found, truth, 3) == pytest.approx((2 / 3 + 0) / 2)
