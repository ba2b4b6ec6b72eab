"""Shared helpers for the GPU parity tests (device plumbing via torch)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from shear_amd import _native as N
from shear_amd import tessa as T


def require_gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU test needs a visible MI355X (run with -m 'not gpu' on CPU machines)")
    N.load()  # the HIP library must be there: no fallback
    return torch.device("cuda:0")


def to_dev_sq8(codes: np.ndarray, scales: np.ndarray, norms: np.ndarray, dim: int | None = None) -> T.Sq8Matrix:
    dev = torch.device("cuda:0")
    return T.Sq8Matrix(torch.from_numpy(np.ascontiguousarray(codes)).to(dev),
                       torch.from_numpy(np.ascontiguousarray(scales, np.float32)).to(dev),
                       torch.from_numpy(np.ascontiguousarray(norms, np.float32)).to(dev),
                       dim if dim is not None else codes.shape[1])


def dev_u32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to("cuda:0")


def run_leaf(sq8: T.Sq8Matrix, gids: np.ndarray, members, offsets, counts, k, executor, debug_rerun_every=0):
    lay = T.LeafLayouts.from_host(np.asarray(members, np.uint32), np.asarray(offsets, np.int64),
                                  np.asarray(counts, np.int64), k)
    ids, d, ctr = T.leaf_topk(sq8, dev_u32(gids), lay, k, executor=executor, debug_rerun_every=debug_rerun_every)
    torch.cuda.synchronize()
    T.raise_on_overflow(ctr, "leaf top-k")
    return (ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), ctr.cpu().numpy())


def assert_same(ids_a, d_a, ids_b, d_b, what=""):
    ids_a = np.asarray(ids_a, np.uint32)
    ids_b = np.asarray(ids_b, np.uint32)
    bad = np.nonzero((ids_a != ids_b) | (np.asarray(d_a, np.float32).view(np.uint32)
                                         != np.asarray(d_b, np.float32).view(np.uint32)))[0]
    if len(bad):
        i = int(bad[0])
        raise AssertionError(f"{what}: {len(bad)} slot mismatches; first at {i}: "
                             f"ids {ids_a[i]} vs {ids_b[i]}, dists {d_a[i]!r} vs {d_b[i]!r}")
