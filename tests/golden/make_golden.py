"""Writes the committed golden fixtures for the oracle (tests/golden/*.npz).

The reference ships no fixtures or golden vectors for its search path, so these are built
here by brute force in numpy, independently of oracle/trident_oracle.c:

  float64 coarse distances -> nprobe smallest by (d, cid)     (np.lexsort)
  float64 distances to every vector of the probed lists -> K smallest by (d, id)

Cases:
  int_ties   integer-valued vectors with duplicated rows and a duplicated centroid: every
             summation order is exact, so the expected values are order independent and the
             fixture pins the (d, id) / (d, cid) tie-breaks.
  float_gmm  Gaussian-mixture floats; the generator checks that no boundary (K-th / nprobe-th)
             has a relative gap below 1e-9, so float64 summation order cannot change the answer.
  short      lists shorter than K and an empty list: missing slots are (+inf, -1).

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def brute(xb, xq, cen, list_ids, nprobe, K):
    q = xq.astype(np.float64)
    cd = ((q[:, None, :] - cen.astype(np.float64)[None]) ** 2).sum(-1)
    B = len(xq)
    probes = np.empty((B, nprobe), np.int32)
    pd = np.empty((B, nprobe))
    out_d = np.full((B, K), np.inf)
    out_i = np.full((B, K), -1, np.int64)
    gaps = []
    for i in range(B):
        o = np.lexsort((np.arange(len(cen)), cd[i]))
        probes[i], pd[i] = o[:nprobe], cd[i, o[:nprobe]]
        if nprobe < len(cen):
            gaps.append((cd[i, o[nprobe]] - cd[i, o[nprobe - 1]]) / max(cd[i, o[nprobe]], 1e-300))
        cand = np.nonzero(np.isin(list_ids, probes[i]))[0]
        if len(cand) == 0:
            continue
        d = ((xb[cand].astype(np.float64) - q[i]) ** 2).sum(1)
        oo = np.lexsort((cand, d))
        if len(oo) > K:
            gaps.append((d[oo[K]] - d[oo[K - 1]]) / max(d[oo[K]], 1e-300))
        oo = oo[:K]
        out_d[i, :len(oo)], out_i[i, :len(oo)] = d[oo], cand[oo]
    return probes, pd, out_d, out_i, np.array(gaps)


def assign(xb, cen):
    return np.argmin(((xb[:, None, :].astype(np.float64) - cen[None]) ** 2).sum(-1), 1).astype(np.int32)


def case_int_ties(rng):
    base = rng.integers(0, 5, size=(300, 16)).astype(np.float32)
    xb = np.concatenate([base, base[:120], base[:40]])
    cen = rng.integers(0, 5, size=(12, 16)).astype(np.float32)
    lid = assign(xb, cen)
    cen[7] = cen[3]
    xq = np.concatenate([rng.integers(0, 5, size=(24, 16)), base[:8]]).astype(np.float32)
    return xb, xq, cen, lid, 4, 10


def case_float_gmm(rng):
    while True:
        centers = rng.uniform(0, 100, size=(8, 16))
        z = rng.integers(0, 8, size=700)
        xb = (centers[z] + 8 * rng.standard_normal((700, 16))).astype(np.float32)
        cen = (centers + rng.standard_normal((8, 16))).astype(np.float32)
        lid = assign(xb, cen)
        zq = rng.integers(0, 8, size=30)
        xq = (centers[zq] + 8 * rng.standard_normal((30, 16))).astype(np.float32)
        gaps = brute(xb, xq, cen, lid, 3, 10)[4]
        if gaps.min() > 1e-9:
            return xb, xq, cen, lid, 3, 10


def case_short(rng):
    xb = rng.integers(0, 9, size=(40, 8)).astype(np.float32)
    cen = rng.integers(0, 9, size=(6, 8)).astype(np.float32)
    lid = assign(xb, cen)
    lid[lid == 2] = 3
    xq = rng.integers(0, 9, size=(10, 8)).astype(np.float32)
    return xb, xq, cen, lid, 2, 30


def main():
    rng = np.random.default_rng(20261201)
    for name, fn in (("int_ties", case_int_ties), ("float_gmm", case_float_gmm), ("short", case_short)):
        xb, xq, cen, lid, nprobe, K = fn(rng)
        probes, pd, d, i, _ = brute(xb, xq, cen, lid, nprobe, K)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, xb=xb, xq=xq, centroids=cen, list_ids=lid, nprobe=nprobe, K=K,
                            probes=probes, probe_d=pd, topk_d=d, topk_i=i)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
