"""The build's terminal-depth retry (rbc_partition.rs:3004-3017, :15066-15115):
a D0 child whose subtree run fails with exactly OVERSIZED_TERMINAL_NODE is run
once more with max_depth raised to 1024.  Tight clusters under a small
max_depth make several children take the retry; the GPU build and the CPU
oracle build (which applies the same rule) write the same `_mem.index`
image and take the same number of retries."""
import pytest
import torch

from gpu_helpers import require_gpu
from oracle import pybuild as PB
from shear_amd import datagen
from shear_amd import pipeline as P

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,comps,sigma,max_depth", [(20000, 4, 0.05, 2), (30000, 2, 0.02, 3)])
def test_terminal_depth_retry_matches_oracle(orc, n, comps, sigma, max_depth):
    gpu = require_gpu()
    x = datagen.gmm_numpy(n, 64, comps, sigma, 5)
    p = P.GraphBuildParams(max_depth=max_depth, c_max=256)
    lead = P.d0_leader_rows(n, 8, p.random_seed)
    sk = P.sketches_of(x, P.sketch_planes(64, p.m_hash_bits, 7))
    built = P.build_graph(torch.from_numpy(x).to(gpu), torch.from_numpy(sk).to(gpu), lead, p)
    cpu = PB.build_graph_cpu(x, sk, lead, p)
    assert cpu["stages"]["terminal_depth_retries"] > 0
    assert built.stages["terminal_depth_retries"] == cpu["stages"]["terminal_depth_retries"]
    assert built.start == cpu["start"]
    assert built.image.cpu().numpy().tobytes() == cpu["image"], "GPU image differs from the CPU build's"
