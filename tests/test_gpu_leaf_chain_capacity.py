"""Leaf top-k on rows that are almost all eps-tie chains, checked against the
oracle bit for bit.

Every row of these leaves holds a run of 36 candidates spaced 0.9e-5 apart
(each adjacent pair is tied under the 2e-5 rule, also across the row itself,
and the run is not a clique), then a wide gap: the select kernel certifies the gap and queues every row
for the chain replay.  In a fresh process the per-device workspace is sized
for this call alone, so its chain pool holds fewer rows than its chain queue;
rows past the pool must take the exact re-run, and the chain kernel must
replay only headers that were written.  The fresh-process case runs in a
child process for that reason.
"""
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

TESTS = Path(__file__).resolve().parent


def chain_case(leaves: int, dim: int = 64):
    """SQ8 rows whose distances inside each 64-row leaf are norm sums: the
    codes are zero, so d(r, c) = n_r + n_c exactly."""
    per = 64
    n = leaves * per
    codes = np.zeros((n, dim), np.int8)
    scales = np.ones(n, np.float32)
    j = np.arange(per)
    leaf_norms = np.where(j < 36, 1.0 + j * 0.9e-5, 3.0 + (j - 36) * 0.01).astype(np.float32)
    norms = np.tile(leaf_norms, leaves)
    gids = np.random.default_rng(leaves).permutation(1 << 20)[:n].astype(np.uint32)
    members = np.arange(n, dtype=np.uint32)
    offs = np.arange(leaves, dtype=np.int64) * per
    counts = np.full(leaves, per, np.int64)
    return codes, scales, norms, gids, members, offs, counts


def run_case(leaves: int) -> dict:
    import torch  # noqa: F401  (device plumbing)

    from gpu_helpers import assert_same, require_gpu, run_leaf, to_dev_sq8
    from oracle import pyoracle as orc
    from shear_amd import _native as N

    require_gpu()
    codes, scales, norms, gids, members, offs, counts = chain_case(leaves)
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, counts, 32)
    sq8 = to_dev_sq8(codes, scales, norms)
    ids, d, ctr = run_leaf(sq8, gids, members, offs, counts, 32, N.EXEC_MFMA)
    assert_same(ids, d, want_ids, want_d, f"chain-heavy leaves={leaves}")
    rows = int(counts.sum())
    assert int(ctr[N.C_LEAF_ROWS]) == rows
    return {"chain": int(ctr[N.C_LEAF_CHAIN_ROWS]), "rerun": int(ctr[N.C_LEAF_FALLBACK_ROWS]), "rows": rows}


def test_chain_case_is_chain_heavy_on_the_oracle(orc):
    """The data really is what the test needs: every row's 32 results come
    from its leaf's tie run, span more than 2e-5 and are followed by a gap
    (checked on the oracle's own output)."""
    codes, scales, norms, gids, members, offs, counts = chain_case(2)
    ids, d = orc.leaf_topk(codes, scales, norms, gids, members, offs, counts, 32)
    d = d.reshape(-1, 32)
    rn = norms[members].astype(np.float64)[:, None]
    cn = d.astype(np.float64) - rn  # the column's norm, up to rounding
    assert np.all(cn < 1.001)  # every result is a run member (norms 1.0 .. 1.000315)
    assert np.all(d.max(axis=1) - d.min(axis=1) > 2e-5)


@pytest.mark.gpu
def test_chain_heavy_leaves_in_process():
    out = run_case(16)
    assert out["chain"] + out["rerun"] == out["rows"]


@pytest.mark.gpu
def test_chain_heavy_leaves_fresh_workspace():
    """1,024 rows in a fresh process: the chain queue holds 4,096 headers but
    the pool only 576 candidate sets."""
    code = ("import json, sys; sys.path[:0] = [%r, %r]; import test_gpu_leaf_chain_capacity as t; "
            "print('RESULT', json.dumps(t.run_case(16)), flush=True)") % (str(TESTS), str(TESTS.parent))
    env = dict(os.environ)
    print("fresh-process chain case: 16 leaves x 64 rows, k=32", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", code], cwd=str(TESTS.parent), env=env,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, f"child failed rc={r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    line = [x for x in r.stdout.splitlines() if x.startswith("RESULT ")]
    assert line, r.stdout
    import json

    out = json.loads(line[-1][len("RESULT "):])
    assert out["rows"] == 1024
    # the pool holds 576 chain sets; the other rows were re-run exactly
    assert out["chain"] <= 576 and out["chain"] + out["rerun"] == 1024, out
