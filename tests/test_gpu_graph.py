"""GPU graph emission (tessa_graph_pack) against the oracle's `_mem.index`
bytes: the reference writer's round-trip and bulk rows, and the graph of
HashPrune reservoirs.  Bar: byte-identical files."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from oracle import pyoracle as O
from shear_amd import graph as G
from shear_amd import hashprune as H
from test_hashprune_oracle import random_stream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _table(rows, stride):
    t = np.full((len(rows), stride), 0xFFFFFFFF, np.uint32)
    for i, r in enumerate(rows):
        t[i, :len(r)] = r
    c = np.array([len(r) for r in rows], np.int32)
    return (torch.from_numpy(t.view(np.int32)).to("cuda:0"), torch.from_numpy(c).to("cuda:0"))


@pytest.mark.parametrize("rows,start,frozen,stride", [
    ([[3, 4], [4], [1, 0, 4], [0], [2, 1]], 17, 0, 4),                       # pipnn_oom_writer.rs:273-300
    ([[(r * 65 + o) for o in range(r % 65)] for r in range(512)], 17, 3, 64),  # :201-220
    ([[] for _ in range(5000)], 0, 0, 8),
    ([], 5, 1, 4),
])
def test_pack_matches_writer_bytes(gpu, rows, start, frozen, stride):
    if not rows:
        t = torch.zeros((0, stride), dtype=torch.int32, device=gpu)
        c = torch.zeros(0, dtype=torch.int32, device=gpu)
    else:
        t, c = _table(rows, stride)
    img = G.pack_mem_index(t, c, start, frozen)
    torch.cuda.synchronize()
    assert img.cpu().numpy().tobytes() == O.graph_bytes(start, frozen, rows)


def test_hashprune_graph_file(gpu, orc, tmp_path):
    rng = np.random.default_rng(4)
    r = random_stream(rng, 3000, 200000, 12, 4000)
    with H.HashPruneReducer(3000, 64) as hp:
        hp.insert(r)
        t, c = hp.neighbors()
        n = G.write_mem_index(tmp_path / "g_mem.index", t, c, start=123)
    wt, _, _, wc = orc.hashprune_reduce(3000, 64, r)
    rows = [wt[p, :wc[p]].tolist() for p in range(3000)]
    data = (tmp_path / "g_mem.index").read_bytes()
    assert n == len(data) and data == O.graph_bytes(123, 0, rows)
