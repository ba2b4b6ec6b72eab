"""Seeded synthetic Gaussian-mixture vectors for the benchmark configurations.

The reference builds on real datasets and ships no generator, so this one is
ours (and unpinned by the reference).  Points are generated component by
component, so rows [c*per, (c+1)*per) belong to component c: "sorted by
component", and leaves cut from consecutive rows are spatially coherent.

* ``gmm_numpy``  CPU, numpy PCG64 -- used by tests and small configs
                 (``gmm_queries_numpy``: held-out queries of the same mixture).
* ``gmm_torch``  GPU, torch Philox on the device -- used for bench-size data
                 (4M x 768 does not fit a host round trip inside a bench run).
* ``c3_torch``   GPU, the in-HBM build configuration: mixture plus uniform
                 outliers, rows in random order (a real dataset is not sorted).
The two generators use different RNG streams; parity tests always feed the
same generated arrays to both sides.
"""
from __future__ import annotations

import numpy as np


def gmm_numpy(n: int, dim: int, components: int, sigma: float, seed: int,
              unit_norm: bool = True) -> np.ndarray:
    rng = np.random.default_rng(seed)
    centers = rng.standard_normal((components, dim)).astype(np.float64)
    per = -(-n // components)
    comp = np.minimum(np.arange(n) // per, components - 1)
    x = centers[comp] + sigma * rng.standard_normal((n, dim))
    if unit_norm:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)


def gmm_queries_numpy(nq: int, dim: int, components: int, sigma: float, seed: int, query_seed: int,
                      unit_norm: bool = True) -> np.ndarray:
    """Held-out queries from the mixture gmm_numpy(seed) draws: the same
    component centres, components picked uniformly and noise drawn from a
    separate generator (query_seed)."""
    centers = np.random.default_rng(seed).standard_normal((components, dim)).astype(np.float64)
    rq = np.random.default_rng(query_seed)
    comp = rq.integers(0, components, nq)
    q = centers[comp] + sigma * rq.standard_normal((nq, dim))
    if unit_norm:
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def gmm_torch(n: int, dim: int, components: int, sigma: float, seed: int, device="cuda",
              unit_norm: bool = True, chunk_rows: int = 1 << 18):
    """Same construction on the GPU, chunked to bound temporary memory."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    centers = torch.randn((components, dim), generator=g, device=device, dtype=torch.float32)
    per = -(-n // components)
    out = torch.empty((n, dim), dtype=torch.float32, device=device)
    for start in range(0, n, chunk_rows):
        end = min(n, start + chunk_rows)
        comp = torch.clamp(torch.arange(start, end, device=device) // per, max=components - 1)
        x = centers[comp] + sigma * torch.randn((end - start, dim), generator=g, device=device)
        if unit_norm:
            x = x / torch.linalg.vector_norm(x, dim=1, keepdim=True)
        out[start:end] = x
    return out



def gmm_queries_torch(nq: int, dim: int, components: int, sigma: float, seed: int, query_seed: int,
                      device="cuda", unit_norm: bool = True):
    """Held-out queries from the mixture gmm_torch(seed) draws: the same
    component centres, components picked uniformly and noise drawn from a
    separate generator (query_seed)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    centers = torch.randn((components, dim), generator=g, device=device, dtype=torch.float32)
    gq = torch.Generator(device=device)
    gq.manual_seed(query_seed)
    comp = torch.randint(0, components, (nq,), generator=gq, device=device)
    q = centers[comp] + sigma * torch.randn((nq, dim), generator=gq, device=device)
    if unit_norm:
        q = q / torch.linalg.vector_norm(q, dim=1, keepdim=True)
    return q

def c3_torch(n: int, dim: int = 768, components: int = 1000, sigma: float = 0.25, outlier_frac: float = 0.05,
             seed: int = 2, device="cuda", chunk_rows: int = 1 << 18):
    """Mixture rows (component centres ~N(0, I), sigma noise) with a fraction of
    U[-1, 1]^dim outliers, unit-normalised, in random row order."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    centers = torch.randn((components, dim), generator=g, device=device, dtype=torch.float32)
    out = torch.empty((n, dim), dtype=torch.float32, device=device)
    for start in range(0, n, chunk_rows):
        end = min(n, start + chunk_rows)
        m = end - start
        comp = torch.randint(0, components, (m,), generator=g, device=device)
        x = centers[comp] + sigma * torch.randn((m, dim), generator=g, device=device)
        noise = torch.rand((m,), generator=g, device=device) < outlier_frac
        u = torch.rand((m, dim), generator=g, device=device) * 2.0 - 1.0
        x = torch.where(noise[:, None], u, x)
        out[start:end] = x / torch.linalg.vector_norm(x, dim=1, keepdim=True)
    return out


def c1_numpy(rows: int = 200_000, nq: int = 1000, dim: int = 128):
    """BASELINE configs[0] (C1): rows x dim f32 from a 64-component isotropic
    mixture, centres ~N(0, I), sigma 0.3, seed 0, not normalised; nq held-out
    queries of the same mixture (query seed 1)."""
    return (gmm_numpy(rows, dim, 64, 0.3, 0, unit_norm=False),
            gmm_queries_numpy(nq, dim, 64, 0.3, 0, 1, unit_norm=False))
