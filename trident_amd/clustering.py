"""Coarse clustering and residual PCA that feed the index layout.

Replaces load_or_train_clustering (benchmarks/phase4a_suite.py:389-439), which calls faiss
k-means (absent here) and numpy eigh.  The outputs have the same meaning: centroids, the list
id of every base vector, residual norms r = |x - c(x)|, and the float64 PCA (mean64, R64) of
the residuals x - c(x) from a 50k sample, eigenvectors by descending eigenvalue.  The
clustering is the index's definition; the search and the oracle consume the same lists, so
exactness does not depend on how well k-means converges.

All work runs as torch ops on the device of ``xb`` (the GPU at scale).
"""
import os
import time

import numpy as np
import torch


def assign(x: torch.Tensor, centroids: torch.Tensor, chunk: int = 1 << 18) -> torch.Tensor:
    """Nearest centroid per row (argmin of |c|^2 - 2 x.c in float32); int64 [N]."""
    cn = (centroids.double() ** 2).sum(1).to(torch.float32)
    ct = centroids.t().contiguous()
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    for s in range(0, x.shape[0], chunk):
        xs = x[s:s + chunk].to(centroids.device, torch.float32)
        out[s:s + chunk] = torch.argmin(cn - 2.0 * (xs @ ct), dim=1).to(x.device)
    return out


def kmeans(x: torch.Tensor, nlist: int, niter: int = 20, seed: int = 0, max_train: int = 0,
           device=None) -> torch.Tensor:
    """Lloyd k-means on a random training subset; empty clusters are re-seeded from random
    training points.  Returns float32 centroids [nlist, D] on ``device``."""
    dev = torch.device(device) if device is not None else x.device
    g = torch.Generator(device="cpu").manual_seed(seed + 1000)
    n = x.shape[0]
    ntrain = min(n, max_train or max(64 * nlist, 65536))
    pick = torch.randperm(n, generator=g)[:ntrain]
    train = x[pick.to(x.device)].to(dev, torch.float32)
    cent = train[torch.randperm(ntrain, generator=g)[:nlist].to(dev)].clone()
    for _ in range(niter):
        a = assign(train, cent)
        sums = torch.zeros_like(cent, dtype=torch.float64).index_add_(0, a, train.double())
        cnt = torch.bincount(a, minlength=nlist)
        empty = cnt == 0
        cent = (sums / cnt.clamp(min=1).unsqueeze(1).double()).to(torch.float32)
        if bool(empty.any()):
            ne = int(empty.sum())
            cent[empty] = train[torch.randint(0, ntrain, (ne,), generator=g).to(dev)]
    return cent.contiguous()


def residual_pca(x: torch.Tensor, centroids: torch.Tensor, list_ids: torch.Tensor, seed: int = 0,
                 sample: int = 50000):
    """float64 PCA of residuals x - c(x) over a random sample: (mean64 [D], R64 [D, D]) with
    eigenvectors in columns by descending eigenvalue (reference :425-434)."""
    n = x.shape[0]
    rng = np.random.default_rng(seed + 42)
    idx = np.sort(rng.choice(n, size=min(sample, n), replace=False))
    it = torch.as_tensor(idx, device=x.device)
    diff = x[it].double().cpu() - centroids[list_ids[it].to(centroids.device)].double().cpu()
    mean64 = diff.mean(0)
    cov = torch.cov(diff.t())
    evals, evecs = torch.linalg.eigh(cov)
    order = torch.argsort(evals, descending=True)
    return mean64.numpy(), evecs[:, order].contiguous().numpy()


def residual_norms(x: torch.Tensor, centroids: torch.Tensor, list_ids: torch.Tensor,
                   chunk: int = 1 << 20) -> torch.Tensor:
    out = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    for s in range(0, x.shape[0], chunk):
        xs = x[s:s + chunk].to(centroids.device).double()
        c = centroids[list_ids[s:s + chunk].to(centroids.device)].double()
        out[s:s + chunk] = torch.sqrt(((xs - c) ** 2).sum(1)).to(torch.float32).to(x.device)
    return out


def train_clustering(xb, nlist: int, seed: int = 0, niter: int = 20, max_train: int = 0,
                     device=None, cache_file: str = ""):
    """(centroids, list_ids, r_vec, mean64, R64, train_time_s), the tuple of
    load_or_train_clustering.  ``cache_file`` (.npz) is written atomically (tmp + os.replace)."""
    if cache_file and os.path.exists(cache_file):
        z = np.load(cache_file, allow_pickle=False)
        return (z["centroids"], z["list_ids"], z["r_vec"], z["mean64"], z["R64"], float(z["train_time_s"]))
    x = xb if isinstance(xb, torch.Tensor) else torch.as_tensor(np.ascontiguousarray(xb, dtype=np.float32))
    dev = torch.device(device) if device is not None else x.device
    if dev.type == "cuda":
        torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    cent = kmeans(x, nlist, niter=niter, seed=seed, max_train=max_train, device=dev)
    lid = assign(x, cent)
    r = residual_norms(x, cent, lid)
    mean64, R64 = residual_pca(x, cent, lid, seed=seed)
    if dev.type == "cuda":
        torch.cuda.synchronize(dev)
    t = time.perf_counter() - t0
    out = (cent.cpu().numpy(), lid.to(torch.int32).cpu().numpy(), r.cpu().numpy(), mean64, R64, t)
    if cache_file:
        tmp = cache_file + f".tmp_{os.getpid()}.npz"
        np.savez(tmp, centroids=out[0], list_ids=out[1], r_vec=out[2], mean64=mean64, R64=R64, train_time_s=t)
        os.replace(tmp, cache_file)
    return out
