"""Seeded synthetic workloads for the five BASELINE.json configurations.

The reference benchmarks real datasets (SIFT, GIST, Deep, BIGANN) that need the network; these
generators produce data of the configured shape and character instead.  Every generator is a
pure function of (seed, sizes, device): torch generators with separate streams for centres,
base and queries.  CPU and GPU draws differ, so a run always checks against the oracle on the
data it generated itself.

cfg1  256-component isotropic Gaussian mixture, centres ~ U[0, 100]^D, sigma = 8.
cfg2  histogram-like integer descriptors: x = clip(round(mu_z + Gamma(0.5, 40)), 0, 255),
      1024 per-cluster bias vectors mu_z ~ U[0, 64]^D, stored as float32.
cfg3  anisotropic Gaussian, eigenvalues lambda_i = i^-1.2 in a random orthogonal basis Q,
      plus a 1024-centre offset mu_z ~ N(0, 0.1^2 I):  x = mu_z + Q (sqrt(lambda) * g).
cfg4  4096 centres mu_z ~ N(0, I); per-centre anisotropic noise: the spectrum
      lambda_i = i^-1 is permuted per centre and applied in a shared random basis,
      x = normalize(mu_z + 0.35 * Q (sqrt(lambda_{pi_z(i)}) * g)).
cfg5  cfg2 at 1e8 rows, generated in chunks with a per-chunk seed.
"""
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch


@dataclass
class Workload:
    name: str
    N: int
    D: int
    B: int
    nlist: int
    nprobe: List[int]
    K: List[int]
    n_centers: int
    integer_valued: bool = False
    extra: Dict = field(default_factory=dict)


CONFIGS = {
    1: Workload("cfg1_gmm_d128", 100_000, 128, 1_000, 256, [16], [10], 256),
    2: Workload("cfg2_hist_d128", 1_000_000, 128, 10_000, 1024, [32, 64, 128], [10], 1024, True),
    3: Workload("cfg3_aniso_d960", 1_000_000, 960, 1_000, 1024, [64], [10, 100], 1024),
    4: Workload("cfg4_norm_d96", 10_000_000, 96, 10_000, 4096, [64], [1, 10, 50, 100], 4096),
    5: Workload("cfg5_hist_d128_100m", 100_000_000, 128, 10_000, 16384, [128], [10], 1024, True),
}


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def _gmm(n, centers, sigma, g, device):
    z = torch.randint(0, centers.shape[0], (n,), generator=g, device=device)
    return centers[z] + sigma * torch.randn((n, centers.shape[1]), generator=g, device=device)


def cfg1(N=100_000, D=128, B=1_000, n_centers=256, seed=0, device="cpu"):
    centers = 100.0 * torch.rand((n_centers, D), generator=_gen(seed * 7919 + 1, device), device=device)
    xb = _gmm(N, centers, 8.0, _gen(seed * 7919 + 2, device), device)
    xq = _gmm(B, centers, 8.0, _gen(seed * 7919 + 3, device), device)
    return xb.float().contiguous(), xq.float().contiguous()


def _hist_rows(n, mu, g, device):
    z = torch.randint(0, mu.shape[0], (n,), generator=g, device=device)
    conc = torch.full((n, mu.shape[1]), 0.5, device=device)
    gam = torch._standard_gamma(conc, generator=g) * 40.0
    return torch.clamp(torch.round(mu[z] + gam), 0.0, 255.0)


def cfg2(N=1_000_000, D=128, B=10_000, n_centers=1024, seed=0, device="cpu", chunk=1 << 22):
    mu = 64.0 * torch.rand((n_centers, D), generator=_gen(seed * 7919 + 11, device), device=device)
    xb = torch.empty((N, D), dtype=torch.float32, device=device)
    for ci, s in enumerate(range(0, N, chunk)):
        e = min(N, s + chunk)
        xb[s:e] = _hist_rows(e - s, mu, _gen(seed * 7919 + 1000 + ci, device), device)
    xq = _hist_rows(B, mu, _gen(seed * 7919 + 13, device), device).float()
    return xb, xq.contiguous()


def _orthogonal(D, g, device):
    a = torch.randn((D, D), generator=g, device=device, dtype=torch.float64)
    q, r = torch.linalg.qr(a)
    return (q * torch.sign(torch.diagonal(r)).unsqueeze(0)).to(torch.float32)


def cfg3(N=1_000_000, D=960, B=1_000, n_centers=1024, seed=0, device="cpu", chunk=1 << 18):
    g0 = _gen(seed * 7919 + 21, device)
    Q = _orthogonal(D, g0, device)
    sl = torch.arange(1, D + 1, device=device, dtype=torch.float32).pow(-0.6)   # sqrt(i^-1.2)
    mu = 0.1 * torch.randn((n_centers, D), generator=g0, device=device)

    def rows(n, g):
        z = torch.randint(0, n_centers, (n,), generator=g, device=device)
        return mu[z] + (torch.randn((n, D), generator=g, device=device) * sl) @ Q.t()

    xb = torch.empty((N, D), dtype=torch.float32, device=device)
    for ci, s in enumerate(range(0, N, chunk)):
        e = min(N, s + chunk)
        xb[s:e] = rows(e - s, _gen(seed * 7919 + 2000 + ci, device))
    xq = rows(B, _gen(seed * 7919 + 23, device))
    return xb, xq.contiguous()


def cfg4(N=10_000_000, D=96, B=10_000, n_centers=4096, seed=0, device="cpu", chunk=1 << 21):
    g0 = _gen(seed * 7919 + 31, device)
    Q = _orthogonal(D, g0, device)
    mu = torch.randn((n_centers, D), generator=g0, device=device)
    sl = torch.arange(1, D + 1, device=device, dtype=torch.float32).pow(-0.5)   # sqrt(i^-1)
    perm = torch.argsort(torch.rand((n_centers, D), generator=g0, device=device), dim=1)
    spec = sl[perm]                                                            # per-centre spectrum

    def rows(n, g):
        z = torch.randint(0, n_centers, (n,), generator=g, device=device)
        x = mu[z] + 0.35 * ((torch.randn((n, D), generator=g, device=device) * spec[z]) @ Q.t())
        return x / x.norm(dim=1, keepdim=True)

    xb = torch.empty((N, D), dtype=torch.float32, device=device)
    for ci, s in enumerate(range(0, N, chunk)):
        e = min(N, s + chunk)
        xb[s:e] = rows(e - s, _gen(seed * 7919 + 3000 + ci, device))
    xq = rows(B, _gen(seed * 7919 + 33, device))
    return xb, xq.contiguous()


def cfg5(N=100_000_000, D=128, B=10_000, n_centers=1024, seed=0, device="cpu", out: Optional[torch.Tensor] = None,
         chunk=1 << 23):
    """cfg2's generator at 1e8 rows, one seed per chunk; ``out`` may be a preallocated buffer."""
    mu = 64.0 * torch.rand((n_centers, D), generator=_gen(seed * 7919 + 11, device), device=device)
    xb = out if out is not None else torch.empty((N, D), dtype=torch.float32, device=device)
    for ci, s in enumerate(range(0, N, chunk)):
        e = min(N, s + chunk)
        xb[s:e] = _hist_rows(e - s, mu, _gen(seed * 7919 + 5000 + ci, device), device).to(xb.device)
    xq = _hist_rows(B, mu, _gen(seed * 7919 + 13, device), device).float()
    return xb, xq.contiguous()


GENERATORS = {1: cfg1, 2: cfg2, 3: cfg3, 4: cfg4, 5: cfg5}


def generate(cfg: int, device="cpu", seed=0, **sizes):
    """(xb, xq) for configuration ``cfg``; keyword sizes (N, D, B, n_centers) override."""
    return GENERATORS[cfg](seed=seed, device=device, **sizes)
