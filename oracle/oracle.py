"""TEST INFRASTRUCTURE ONLY -- the parity checker for the lossless IVF query path.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this
module; the product (``trident_amd``) never does.

Two independent restatements of the reference's exact-search semantics live here:

* ctypes wrappers over ``trident_oracle.c`` (fast, OpenMP): the canonical float64
  oracle (probe + exhaustive IVF, (d, id) tie-break) and the FP32 IVF-Flat CPU baseline
  ``omp_cpu_ivfflat_f32`` (benchmarks/phase8_ooc_100m_4080.py:141-204);
* pure numpy brute force for small inputs (``np_coarse_probe``, ``np_ivf_exact``) that
  follows the float64 audit (benchmarks/phase4b_suite.py:185-219) with the
  ``np.lexsort((ids, d))`` tie-break of benchmarks/phase3a_lossless_audit.py:62.  The
  numpy path sums in a different order than the C path, so the two agree bit for bit only
  where every order is exact (integer-valued data) and otherwise to float64 rounding;
  that independence is what pins the C restatement.

``audit`` restates the float64 audit taxonomy of
benchmarks/phase3a_lossless_audit.py:76-129 (exact tie / f32 rounding / true miss).
"""
import ctypes
import os

import numpy as np

from . import build as _build

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = _build.build(force=False)
        L = ctypes.CDLL(path)
        i64, i32, dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_double
        P = ctypes.c_void_p
        L.oracle_coarse_probe.argtypes = [P, i64, i32, P, i32, i32, P, P, i32]
        L.oracle_ivf_exact.argtypes = [P, i64, i32, P, i32, P, P, P, i32, P, P, i32]
        L.oracle_ivfflat_f32.argtypes = [P, i64, i32, P, i32, P, P, P, i32, P, P, i32]
        L.oracle_ivf_exact_cm.argtypes = [P, i64, i32, P, i32, P, P, P, i32, i32, P, P, i32]
        L.oracle_ivf_exact_cm.restype = i32
        L.oracle_pair_dists.argtypes = [P, i32, P, P, P, i64, P]
        L.oracle_rotate_query.argtypes = [P, i32, i32, P, i32, P, P]
        L.oracle_rotate_query.restype = None
        L.oracle_ivf_sq8.argtypes = [P, i64, i32, i32, P, P, i32, P, i32, i32, P, P, i32, P, P, P, P,
                                     i32, P, i32, i32, i32, i32, P, P, i32]
        L.oracle_ivf_sq8.restype = i32
        L.oracle_dist_f64.argtypes = [P, P, i32]
        L.oracle_dist_f64.restype = dbl
        L.oracle_max_threads.restype = i32
        for f in (L.oracle_coarse_probe, L.oracle_ivf_exact, L.oracle_ivfflat_f32, L.oracle_pair_dists):
            f.restype = i32
        _LIB = L
    return _LIB


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)


def coarse_probe(xq, centroids, nprobe, threads=0):
    """float64 coarse probe: (cids int32 [B, nprobe], d float64 [B, nprobe]) by (d, cid)."""
    xq, pq = _c(xq, np.float32)
    cen, pc = _c(centroids, np.float32)
    B, D = xq.shape
    nlist = cen.shape[0]
    cids = np.empty((B, nprobe), np.int32)
    d = np.empty((B, nprobe), np.float64)
    rc = lib().oracle_coarse_probe(pq, B, D, pc, nlist, nprobe, cids.ctypes.data, d.ctypes.data,
                                   threads or default_threads())
    if rc:
        raise ValueError("oracle_coarse_probe: bad arguments")
    return cids, d


def ivf_exact(xq, probe_cids, vec_off, xb_sorted, orig_ids, K, threads=0):
    """Exhaustive float64 IVF: (d float64 [B, K], ids int64 [B, K]); missing = (+inf, -1)."""
    xq, pq = _c(xq, np.float32)
    pcid, ppc = _c(probe_cids, np.int32)
    voff, pvo = _c(vec_off, np.int32)
    xb, pxb = _c(xb_sorted, np.float32)
    oid, poi = _c(orig_ids, np.int32)
    B, D = xq.shape
    d = np.empty((B, K), np.float64)
    ids = np.empty((B, K), np.int64)
    rc = lib().oracle_ivf_exact(pq, B, D, ppc, pcid.shape[1], pvo, pxb, poi, K, d.ctypes.data,
                                ids.ctypes.data, threads or default_threads())
    if rc:
        raise ValueError("oracle_ivf_exact: bad arguments")
    return d, ids


def ivf_exact_cm(xq, probe_cids, vec_off, xb_sorted, orig_ids, K, threads=0):
    """``ivf_exact``'s result computed cluster-major (each probed list read once for every query
    that probes it): the fast form for large batches whose queries share clusters."""
    xq, pq = _c(xq, np.float32)
    pcid, ppc = _c(probe_cids, np.int32)
    voff, pvo = _c(vec_off, np.int32)
    xb, pxb = _c(xb_sorted, np.float32)
    oid, poi = _c(orig_ids, np.int32)
    B, D = xq.shape
    d = np.empty((B, K), np.float64)
    ids = np.empty((B, K), np.int64)
    rc = lib().oracle_ivf_exact_cm(pq, B, D, ppc, pcid.shape[1], pvo, pxb, poi, len(voff) - 1, K,
                                   d.ctypes.data, ids.ctypes.data, threads or default_threads())
    if rc == -2:
        raise MemoryError("oracle_ivf_exact_cm: pair lists do not fit in host memory")
    if rc:
        raise ValueError("oracle_ivf_exact_cm: bad arguments")
    return d, ids


def ivfflat_f32(xq, probe_cids, vec_off, xb_sorted, orig_ids, K, threads=0):
    """The reference CPU IVF-Flat baseline (FP32, OpenMP): (d float32 [B, K], ids int64)."""
    xq, pq = _c(xq, np.float32)
    pcid, ppc = _c(probe_cids, np.int32)
    voff, pvo = _c(vec_off, np.int32)
    xb, pxb = _c(xb_sorted, np.float32)
    oid, poi = _c(orig_ids, np.int32)
    B, D = xq.shape
    d = np.empty((B, K), np.float32)
    ids = np.empty((B, K), np.int64)
    rc = lib().oracle_ivfflat_f32(pq, B, D, ppc, pcid.shape[1], pvo, pxb, poi, K, d.ctypes.data,
                                  ids.ctypes.data, threads or default_threads())
    if rc:
        raise ValueError("oracle_ivfflat_f32: bad arguments")
    return d, ids


def pair_dists(xq, xb_sorted, qids, spos):
    """Canonical float64 distance for explicit (query, sorted row) pairs."""
    xq, pq = _c(xq, np.float32)
    xb, pxb = _c(xb_sorted, np.float32)
    qi, pqi = _c(qids, np.int32)
    sp, psp = _c(spos, np.int64)
    out = np.empty(len(qi), np.float64)
    lib().oracle_pair_dists(pq, xq.shape[1], pxb, pqi, psp, len(qi), out.ctypes.data)
    return out


def sq8_mode_plan(mode, B, K, nprobe, rerank_m):
    """(p_init, k_p1, k_p2, M) of modes 0 / 1: the reference's two-pass split
    (src/trident_v4_kernels.cu:1264-1276), per-pair list lengths (:1439-1443, K_LOC cap :576)
    and rerank length (:1071-1073).  Mode 1 keeps K per pair: the reference's K_LOC = 10 gives
    the same top-K for every K <= 10, the only K its merge returns (:984)."""
    if mode == 0:
        if nprobe <= 1 or (B == 1 and rerank_m == 0):
            p_init = 0
        elif (rerank_m > 20 or K > 10) and nprobe >= 4:
            p_init = 2
        else:
            p_init = 1
    elif nprobe <= 1:
        p_init = 0
    elif B == 1 and K <= 10:
        p_init = 1
    else:
        p_init = 2 if nprobe <= 16 else 3
    eff = max(rerank_m, K) if (mode == 0 and rerank_m > 0) else 0
    if eff:
        k1 = min(eff, 128)
        k2 = min(eff, max(K, max(16, (eff + nprobe - 1) // nprobe + 8)), 200)
        return p_init, k1, k2, min(eff, 200)
    return p_init, K, K, 0


def rotate_query(q, W_combined, b_combined, nlist, D_pad):
    """q R + b as the SQ8 modes compute it (float64 fma chain per column)."""
    q, pq = _c(q, np.float32)
    W, pw = _c(W_combined, np.float32)
    b, pb = _c(b_combined.reshape(-1), np.float32)
    out = np.empty(D_pad, np.float64)
    lib().oracle_rotate_query(pq, q.shape[0], D_pad, pw, nlist, pb, out.ctypes.data)
    return out


def ivf_sq8(xq, probe_cids, p_init, ix, K, k_p1, k_p2, M, threads=0):
    """Modes 0 / 1 (see trident_oracle.c): (d float32 [B, K], ids int64 [B, K]).  ``ix`` holds
    numpy copies of the index tensors: W_combined, b_combined, nlist, D_pad, vec_off, tile_off,
    T, sq8_packed, tile_oids, vmin, delta, per_cluster, xb_sorted."""
    xq, pq = _c(xq, np.float32)
    pcid, ppc = _c(probe_cids, np.int32)
    W, pw = _c(ix["W_combined"], np.float32)
    b, pb = _c(np.asarray(ix["b_combined"]).reshape(-1), np.float32)
    voff, pvo = _c(ix["vec_off"], np.int32)
    toff, pto = _c(ix["tile_off"], np.int32)
    codes, pcd = _c(np.asarray(ix["sq8_packed"]).view(np.uint32), np.uint32)
    toid, pti = _c(ix["tile_oids"], np.int32)
    vmin, pvm = _c(ix["vmin"], np.float32)
    dlt, pdl = _c(ix["delta"], np.float32)
    xb, pxb = _c(ix["xb_sorted"], np.float32)
    B, D = xq.shape
    d = np.empty((B, K), np.float32)
    ids = np.empty((B, K), np.int64)
    rc = lib().oracle_ivf_sq8(pq, B, D, int(ix["D_pad"]), pw, pb, int(ix["nlist"]), ppc, pcid.shape[1],
                              int(p_init), pvo, pto, int(ix["T"]), pcd, pti, pvm, pdl,
                              int(ix["per_cluster"]), pxb, K, int(k_p1), int(k_p2), int(M),
                              d.ctypes.data, ids.ctypes.data, threads or default_threads())
    if rc:
        raise ValueError("oracle_ivf_sq8: bad arguments")
    return d, ids


# ----------------------------------------------------------------------------------------
# numpy brute force (small inputs only)
# ----------------------------------------------------------------------------------------
def np_coarse_probe(xq, centroids, nprobe):
    q = xq.astype(np.float64)
    c = centroids.astype(np.float64)
    d = ((q[:, None, :] - c[None, :, :]) ** 2).sum(axis=2)
    B, nlist = d.shape
    cids = np.empty((B, nprobe), np.int32)
    dd = np.empty((B, nprobe), np.float64)
    ar = np.arange(nlist)
    for i in range(B):
        o = np.lexsort((ar, d[i]))[:nprobe]
        cids[i] = o
        dd[i] = d[i, o]
    return cids, dd


def np_ivf_exact(xq, xb, list_ids, probe_cids, K):
    """Brute force over the ORIGINAL-order base: gather every vector whose list is probed."""
    q64 = xq.astype(np.float64)
    B = xq.shape[0]
    out_d = np.full((B, K), np.inf)
    out_i = np.full((B, K), -1, np.int64)
    for i in range(B):
        cand = np.nonzero(np.isin(list_ids, probe_cids[i]))[0]
        if len(cand) == 0:
            continue
        d = ((xb[cand].astype(np.float64) - q64[i]) ** 2).sum(axis=1)
        o = np.lexsort((cand, d))[:K]
        out_d[i, :len(o)] = d[o]
        out_i[i, :len(o)] = cand[o]
    return out_d, out_i


def audit(pred_ids, ref_ids, xb, xq):
    """Float64 audit of a predicted id list against the reference list (restates
    audit_predictions, benchmarks/phase3a_lossless_audit.py:76-129, for any K).

    Per query, the ids in only one of the two lists are paired in order of their float64
    distance and each pair is classified as an exact tie (|dp - dr| <= 1e-12 max(1, dr)), an
    FP32 rounding difference (relative <= 1e-5) or a true miss; ids that cannot be paired (a
    list shorter than the other, -1 slots) count as true misses.  ``xb`` is indexed by id."""
    Q = len(ref_ids)
    K = int(np.asarray(ref_ids).shape[1]) if Q else 0
    res = dict(diff_slots=0, exact_tie=0, f32_rounding=0, true_miss=0, max_rel=0.0,
               total_slots=Q * K, strict_id_hits=0, queries_strict=0, queries_no_miss=0)
    for q in range(Q):
        sp = set(int(i) for i in pred_ids[q] if i >= 0)
        sr = set(int(i) for i in ref_ids[q] if i >= 0)
        res["strict_id_hits"] += len(sp & sr)
        if sp == sr:
            res["queries_strict"] += 1
            res["queries_no_miss"] += 1
            continue
        qv = xq[q].astype(np.float64)
        dist = lambda i: float(((xb[i].astype(np.float64) - qv) ** 2).sum())
        miss = sorted(sr - sp, key=dist)
        extra = sorted(sp - sr, key=dist)
        q_miss = abs(len(miss) - len(extra))
        for r, p in zip(miss, extra):
            dr, dp = dist(r), dist(p)
            rel = abs(dp - dr) / max(dr, 1e-12)
            res["max_rel"] = max(res["max_rel"], rel)
            res["diff_slots"] += 1
            if abs(dp - dr) <= 1e-12 * max(1.0, dr):
                res["exact_tie"] += 1
            elif rel <= 1e-5:
                res["f32_rounding"] += 1
            else:
                q_miss += 1
        res["true_miss"] += q_miss
        res["queries_no_miss"] += q_miss == 0
    slots = max(res["total_slots"], 1)
    res["strict_id_overlap_pct"] = 100.0 * res["strict_id_hits"] / slots
    res["lossless_no_miss_pct"] = 100.0 * res["queries_no_miss"] / max(Q, 1)
    return res
