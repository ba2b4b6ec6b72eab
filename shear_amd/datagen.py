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
* ``MixtureSpec`` GPU, chunked: the C3 / C4 / C5 mixtures (uniform or Zipf
                 component weights, one sigma or a per-component sigma range,
                 uniform outliers); every chunk of rows is drawn from its own
                 generator, so any chunk can be regenerated on its own (a
                 150M x 768 set is never held as f32).
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


class MixtureSpec:
    """A seeded Gaussian mixture generated in independent chunks.

    Component centres ~N(0, I) (dim); component c has noise sigma_c (a fixed
    sigma, or uniform in [sigma_lo, sigma_hi] per component); weights uniform
    or Zipf(s) over components in random rank order; a fraction of rows are
    U[-1, 1]^dim outliers; rows unit-normalised when asked.  Rows
    [i * chunk_rows, (i + 1) * chunk_rows) come from generator seed
    (seed, i), so chunk i is the same whenever it is drawn."""

    def __init__(self, n: int, dim: int, components: int, sigma=0.25, outlier_frac: float = 0.0, seed: int = 0,
                 zipf_s: float | None = None, unit_norm: bool = True, chunk_rows: int = 1 << 20):
        self.n, self.dim, self.components = int(n), int(dim), int(components)
        self.sigma, self.outlier_frac, self.seed = sigma, float(outlier_frac), int(seed)
        self.zipf_s, self.unit_norm, self.chunk_rows = zipf_s, unit_norm, int(chunk_rows)
        self._dev_cache = {}

    @property
    def chunks(self) -> int:
        return -(-self.n // self.chunk_rows)

    def _params(self, device):
        import torch

        key = str(device)
        if key not in self._dev_cache:
            g = torch.Generator(device="cpu")
            g.manual_seed(self.seed)
            centers = torch.randn((self.components, self.dim), generator=g, dtype=torch.float32)
            if isinstance(self.sigma, (tuple, list)):
                lo, hi = self.sigma
                sig = lo + (hi - lo) * torch.rand(self.components, generator=g, dtype=torch.float32)
            else:
                sig = torch.full((self.components,), float(self.sigma), dtype=torch.float32)
            if self.zipf_s is not None:
                w = 1.0 / torch.arange(1, self.components + 1, dtype=torch.float64) ** float(self.zipf_s)
                w = w[torch.randperm(self.components, generator=g)]
            else:
                w = torch.ones(self.components, dtype=torch.float64)
            self._dev_cache[key] = (centers.to(device), sig.to(device), (w / w.sum()).to(device))
        return self._dev_cache[key]

    def chunk(self, i: int, device="cuda"):
        """f32 [rows, dim] device tensor of chunk i."""
        import torch

        centers, sig, w = self._params(device)
        start = i * self.chunk_rows
        m = min(self.n, start + self.chunk_rows) - start
        g = torch.Generator(device=device)
        g.manual_seed((self.seed * 1000003 + i) & ((1 << 63) - 1))
        if self.zipf_s is not None:
            comp = torch.multinomial(w, m, replacement=True, generator=g)
        else:
            comp = torch.randint(0, self.components, (m,), generator=g, device=device)
        x = centers[comp] + sig[comp, None] * torch.randn((m, self.dim), generator=g, device=device)
        if self.outlier_frac > 0.0:
            noise = torch.rand((m,), generator=g, device=device) < self.outlier_frac
            u = torch.rand((m, self.dim), generator=g, device=device) * 2.0 - 1.0
            x = torch.where(noise[:, None], u, x)
        if self.unit_norm:
            x = x / torch.linalg.vector_norm(x, dim=1, keepdim=True)
        return x

    def rows(self, device="cuda"):
        """The whole set as one f32 device tensor (when it fits)."""
        import torch

        out = torch.empty((self.n, self.dim), dtype=torch.float32, device=device)
        for i in range(self.chunks):
            out[i * self.chunk_rows: i * self.chunk_rows + min(self.chunk_rows, self.n - i * self.chunk_rows)] = \
                self.chunk(i, device)
        return out

    def queries(self, nq: int, query_seed: int, device="cuda"):
        """Held-out queries of the mixture (no outliers), from their own generator."""
        import torch

        centers, sig, w = self._params(device)
        g = torch.Generator(device=device)
        g.manual_seed(query_seed)
        comp = torch.multinomial(w, nq, replacement=True, generator=g)
        q = centers[comp] + sig[comp, None] * torch.randn((nq, self.dim), generator=g, device=device)
        if self.unit_norm:
            q = q / torch.linalg.vector_norm(q, dim=1, keepdim=True)
        return q


def c3_spec(n: int = 10_000_000) -> MixtureSpec:
    """BASELINE configs[2] (C3): 1,000 components, sigma 0.25, 5 % uniform outliers, seed 2, unit-normalised."""
    return MixtureSpec(n, 768, 1000, 0.25, 0.05, 2)


def c4_spec(n: int = 35_000_000) -> MixtureSpec:
    """BASELINE configs[3] (C4): 4,000 components with Zipf(1.1) sizes, seed 3, unit-normalised
    (sigma not given by the config: 0.25, as C3)."""
    return MixtureSpec(n, 768, 4000, 0.25, 0.0, 3, zipf_s=1.1)


def c5_spec(n: int = 150_000_000) -> MixtureSpec:
    """BASELINE configs[4] (C5): 16,000 components, sigma uniform in [0.15, 0.4] per component, seed 4,
    unit-normalised."""
    return MixtureSpec(n, 768, 16000, (0.15, 0.4), 0.0, 4)
