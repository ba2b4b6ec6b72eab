"""GPU parity of the final RobustPrune (tessa_robust_prune) with the CPU
oracle's restatement of final_prune_pipnn / occlude_list
(shear-core/src/index/inmem_index/pipnn_builder.rs:287-330,
algorithm/prune/prune.rs:17-214).  Bar: every row's ids and count identical."""
import numpy as np
import pytest
import torch

from gpu_helpers import require_gpu
from shear_amd import _native as N
from shear_amd import graph as G
from shear_amd import hashprune as H
from test_hashprune_oracle import random_stream
from test_gpu_search import random_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def _prune(gpu, x, t, c, **kw):
    out, cnt = G.robust_prune(torch.from_numpy(x).to(gpu), torch.from_numpy(t.view(np.int32)).to(gpu),
                              torch.from_numpy(c.astype(np.int32)).to(gpu), **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32), cnt.cpu().numpy().view(np.uint32)


def _same(got, want, what):
    go, gc = got
    wo, wc = want
    bad = np.nonzero((gc != wc) | np.any(go != wo, 1))[0]
    assert len(bad) == 0, f"{what}: rows {bad[:8]} differ, e.g. got {go[bad[0]][:gc[bad[0]]]} want {wo[bad[0]][:wc[bad[0]]]}"


@pytest.mark.parametrize("seed,n,dim,stride,kw", [
    (1, 2000, 16, 64, {}),
    (2, 1500, 128, 100, dict(max_degree=32)),
    (3, 1000, 7, 256, dict(max_degree=256, max_occlusion=200)),
    (4, 3000, 24, 40, dict(alpha=1.5, saturate=True)),
    (5, 800, 3, 30, dict(alpha=1.0, max_degree=8)),
    (6, 500, 64, 64, dict(alpha=2.0, max_occlusion=10, saturate=True)),
])
def test_random_tables_match_oracle(gpu, orc, seed, n, dim, stride, kw):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    t, c = random_graph(rng, n, stride)
    t[::9, 0] = np.arange(0, n, 9)  # self-loops
    _same(_prune(gpu, x, t, c, **kw), orc.robust_prune(x, t, c, **kw), f"seed {seed}")


def test_coincident_points_and_ties(gpu, orc):
    rng = np.random.default_rng(7)
    x = rng.integers(0, 3, (600, 4)).astype(np.float32)  # many zero and equal distances
    t, c = random_graph(rng, 600, 48)
    _same(_prune(gpu, x, t, c), orc.robust_prune(x, t, c), "ties")


def test_hashprune_rows(gpu, orc):
    rng = np.random.default_rng(8)
    n, dim = 700, 32
    x = rng.standard_normal((n, dim)).astype(np.float32)
    r = random_stream(rng, n, 50000, 12, 5000)
    r["dst"] = r["dst"] % n
    with H.HashPruneReducer(n, 64) as hp:
        hp.insert(r)
        tt, cc = hp.neighbors()
        out, cnt = G.robust_prune(torch.from_numpy(x).to(gpu), tt, cc)
        torch.cuda.synchronize()
        th, ch = tt.cpu().numpy().view(np.uint32), cc.cpu().numpy().view(np.uint32)
    _same((out.cpu().numpy().view(np.uint32), cnt.cpu().numpy().view(np.uint32)), orc.robust_prune(x, th, ch),
          "hashprune rows")


def test_limits(gpu):
    x = torch.zeros((4, 4), device=gpu)
    t = torch.zeros((4, 300), dtype=torch.int32, device=gpu)
    c = torch.zeros(4, dtype=torch.int32, device=gpu)
    with pytest.raises(N.TessaError, match="row_stride 300"):
        G.robust_prune(x, t, c)
