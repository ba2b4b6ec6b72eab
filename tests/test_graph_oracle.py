"""`_mem.index` layout (oracle graph_bytes and the host reader), pinned by the
reference writer's round-trip rows (pipnn_oom_writer.rs:273-300), whose bytes
are worked out by hand below, and by the size/degree invariants of its bulk
test (:201-220)."""
import numpy as np

from oracle import pyoracle as O
from shear_amd import graph as G


def test_round_trip_rows_by_hand():
    rows = [[3, 4], [4], [1, 0, 4], [0], [2, 1]]
    b = O.graph_bytes(17, 0, rows)
    # 24-byte header + (1+2)+(1+1)+(1+3)+(1+1)+(1+2) = 14 words
    want = (np.array([80], "<u8").tobytes() + np.array([3, 17], "<u4").tobytes() + np.array([0], "<u8").tobytes()
            + np.array([2, 3, 4, 1, 4, 3, 1, 0, 4, 1, 0, 2, 2, 1], "<u4").tobytes())
    assert b == want
    start, frozen, maxd, back = G.read_mem_index(b)
    assert (start, frozen, maxd) == (17, 0, 3)
    assert [r.tolist() for r in back] == rows


def test_bulk_rows_invariants():
    rows = [[(r * 65 + o) & 0xFFFFFFFF for o in range(r % 65)] for r in range(512)]
    b = O.graph_bytes(17, 3, rows)
    start, frozen, maxd, back = G.read_mem_index(b)
    assert (start, frozen, maxd) == (17, 3, 64)
    assert len(b) == 24 + 4 * sum(1 + len(r) for r in rows)
    assert [r.tolist() for r in back] == rows


def test_empty_graph():
    b = O.graph_bytes(0, 0, [])
    assert len(b) == 24 and G.read_mem_index(b)[3] == []
