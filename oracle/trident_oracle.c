/*
 * trident_oracle.c -- TEST INFRASTRUCTURE ONLY (the parity checker, never the product).
 *
 * CPU restatement of the reference's lossless-IVF query semantics, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product path
 * (trident_amd/) never links, loads or calls anything in this directory.
 *
 * Functions and the reference behaviour each one restates:
 *
 *   oracle_dist_f64        canonical float64 squared L2: t = (double)x_d - (double)q_d,
 *                          acc = fma(t, t, acc) for d = 0..D-1 in order.  The float64
 *                          audit computes sum((x64 - q64)^2)
 *                          (benchmarks/phase3a_lossless_audit.py:56-58,
 *                          benchmarks/phase4b_suite.py:211-213); fixing the summation
 *                          order makes the GPU and this oracle bit-identical.
 *   oracle_coarse_probe    float64 coarse distances to every centroid, nprobe smallest
 *                          ordered by (d, cid): benchmarks/phase4b_suite.py:190-195
 *                          (float64 coarse step) with the cid tie-break of
 *                          src/trident_v4_kernels.cu:117-161.
 *   oracle_ivf_exact       exhaustive float64 IVF over the probed lists, top-K by
 *                          (d, id) lexicographic: benchmarks/phase4b_suite.py:197-219,
 *                          tie-break of benchmarks/phase3a_lossless_audit.py:62 and
 *                          insert_topk (src/trident_v4_kernels.cu:19-60).
 *   oracle_ivf_exact_cm    the same result computed cluster-major (each probed list read
 *                          once for all the queries that probe it), for large batches.
 *   oracle_ivfflat_f32     the reference CPU baseline omp_cpu_ivfflat_f32
 *                          (benchmarks/phase8_ooc_100m_4080.py:141-204): FP32 direct
 *                          sum with an OpenMP SIMD reduction and (d, id) insertion.
 *   oracle_rotate_query    the query rotation q -> q R + b of the SQ8 modes as one float64
 *                          fma chain per column over d in order, plus b_j (the reference
 *                          computes it with its float32 GEMM, src/trident_v4_kernels.cu:
 *                          1241-1243; this path fixes the float64 chain instead).
 *   oracle_ivf_sq8         modes 1 (K1) and 0 (K0 / CM-SQ8+RR),
 *                          src/trident_v4_kernels.cu:529-962 and :1044-1170: every probed
 *                          vector's SQ8 reconstruction distance acc_hat = sum_d fmaf(a_d, a_d,
 *                          acc), a_d = fmaf(code_d, delta_d, fl32(vmin_d - q_rot,d)), dims in
 *                          order; each (query, cluster) pair keeps its k_pass best by
 *                          (acc_hat, original id) (K_LOC, :576), the pool's best M (mode 0,
 *                          :1071-1073) are reranked by the canonical float64 distance and
 *                          the top-K by (d, id) returned; without a rerank the top-K by
 *                          (acc_hat, id), acc_hat as the distance.
 *
 * Parity pins: see the checks in tests/test_oracle.py (brute force in numpy on tiny
 * inputs, committed golden fixtures, integer-valued data where every summation order is
 * exact, and planted-mistake checks).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

double oracle_dist_f64(const float* x, const float* q, int D) {
    double acc = 0.0;
    for (int d = 0; d < D; ++d) {
        double t = (double)x[d] - (double)q[d];
        acc = fma(t, t, acc);
    }
    return acc;
}

/* oracle_dist_f64 of 8 consecutive rows (row stride D): the same per-row fma chain in dimension
 * order, eight independent chains interleaved so that the FMA units are not left waiting on one
 * chain's latency.  Bit-identical to eight oracle_dist_f64 calls. */
static inline void oracle_dist8_f64(const float* x, const float* q, int D, double* out) {
    double a[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    for (int d = 0; d < D; ++d) {
        const double qd = (double)q[d];
        for (int r = 0; r < 8; ++r) {
            const double t = (double)x[(int64_t)r * D + d] - qd;
            a[r] = fma(t, t, a[r]);
        }
    }
    for (int r = 0; r < 8; ++r) out[r] = a[r];
}

/* (d, id) strictly-less, the ordering contract of insert_topk. */
static inline int lex_less(double da, int64_t ia, double db, int64_t ib) {
    return (da < db) || (da == db && ia < ib);
}

/* Insert (d, id) into a list sorted ascending by (d, id) of length K; the list is
 * pre-filled with (+inf, INT64_MAX) sentinels. */
static inline void insert_sorted(double* ld, int64_t* li, int K, double d, int64_t id) {
    if (!lex_less(d, id, ld[K - 1], li[K - 1])) return;
    int j = K - 1;
    while (j > 0 && lex_less(d, id, ld[j - 1], li[j - 1])) {
        ld[j] = ld[j - 1];
        li[j] = li[j - 1];
        --j;
    }
    ld[j] = d;
    li[j] = id;
}

int oracle_coarse_probe(const float* xq, int64_t B, int D, const float* centroids, int nlist,
                        int nprobe, int32_t* out_cids, double* out_d, int nthreads) {
    if (nprobe < 1 || nprobe > nlist || D < 1) return -1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        double* ld = (double*)malloc(sizeof(double) * (size_t)nprobe);
        int64_t* li = (int64_t*)malloc(sizeof(int64_t) * (size_t)nprobe);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (int64_t q = 0; q < B; ++q) {
            const float* qv = xq + q * (int64_t)D;
            for (int j = 0; j < nprobe; ++j) { ld[j] = INFINITY; li[j] = INT64_MAX; }
            for (int c = 0; c < nlist; ++c) {
                double d = oracle_dist_f64(centroids + (int64_t)c * D, qv, D);
                insert_sorted(ld, li, nprobe, d, c);
            }
            for (int j = 0; j < nprobe; ++j) {
                out_cids[q * nprobe + j] = (int32_t)li[j];
                if (out_d) out_d[q * nprobe + j] = ld[j];
            }
        }
        free(ld);
        free(li);
    }
    return 0;
}

int oracle_ivf_exact(const float* xq, int64_t B, int D, const int32_t* probe_cids, int nprobe,
                     const int32_t* vec_off, const float* xb_sorted, const int32_t* orig_ids,
                     int K, double* out_d, int64_t* out_i, int nthreads) {
    if (K < 1 || D < 1) return -1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        double* ld = (double*)malloc(sizeof(double) * (size_t)K);
        int64_t* li = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t q = 0; q < B; ++q) {
            const float* qv = xq + q * (int64_t)D;
            for (int j = 0; j < K; ++j) { ld[j] = INFINITY; li[j] = INT64_MAX; }
            for (int p = 0; p < nprobe; ++p) {
                int32_t c = probe_cids[q * nprobe + p];
                if (c < 0) continue;
                int64_t v = vec_off[c];
                const int64_t ve = vec_off[c + 1];
                for (; v + 8 <= ve; v += 8) {
                    double d8[8];
                    oracle_dist8_f64(xb_sorted + v * D, qv, D, d8);
                    for (int r = 0; r < 8; ++r) insert_sorted(ld, li, K, d8[r], (int64_t)orig_ids[v + r]);
                }
                for (; v < ve; ++v) {
                    double d = oracle_dist_f64(xb_sorted + v * D, qv, D);
                    insert_sorted(ld, li, K, d, (int64_t)orig_ids[v]);
                }
            }
            for (int j = 0; j < K; ++j) {
                int valid = li[j] != INT64_MAX;
                out_d[q * K + j] = valid ? ld[j] : INFINITY;
                out_i[q * K + j] = valid ? li[j] : -1;
            }
        }
        free(ld);
        free(li);
    }
    return 0;
}

int oracle_ivfflat_f32(const float* xq, int64_t B, int D, const int32_t* probe_cids, int nprobe,
                       const int32_t* vec_off, const float* xb_sorted, const int32_t* orig_ids,
                       int K, float* out_d, int64_t* out_i, int nthreads) {
    if (K < 1 || D < 1) return -1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int64_t q = 0; q < B; ++q) {
        const float* qr = xq + q * (int64_t)D;
        float* td = out_d + q * K;
        int64_t* ti = out_i + q * K;
        for (int j = 0; j < K; ++j) { td[j] = INFINITY; ti[j] = -1; }
        for (int p = 0; p < nprobe; ++p) {
            int32_t c = probe_cids[q * nprobe + p];
            if (c < 0) continue;
            for (int64_t v = vec_off[c]; v < vec_off[c + 1]; ++v) {
                const float* br = xb_sorted + v * D;
                float sum = 0.0f;
#ifdef _OPENMP
#pragma omp simd reduction(+ : sum)
#endif
                for (int d = 0; d < D; ++d) {
                    float diff = qr[d] - br[d];
                    sum += diff * diff;
                }
                int64_t id = (int64_t)orig_ids[v];
                /* insertion with the (d, id) tie-break; empty slots hold (+inf, -1) */
                if (sum < td[K - 1] || (sum == td[K - 1] && id < ti[K - 1])) {
                    td[K - 1] = sum;
                    ti[K - 1] = id;
                    for (int j = K - 1; j > 0; --j) {
                        int swap = td[j] < td[j - 1] || (td[j] == td[j - 1] && ti[j] < ti[j - 1]);
                        if (!swap) break;
                        float tdv = td[j]; td[j] = td[j - 1]; td[j - 1] = tdv;
                        int64_t tiv = ti[j]; ti[j] = ti[j - 1]; ti[j - 1] = tiv;
                    }
                }
            }
        }
    }
    return 0;
}

/* q R + b for one query: xr[j] = fma chain over d of (double)q_d * (double)W[d][nlist + j], then
 * + (double)b[nlist + j]; j < D_pad. */
void oracle_rotate_query(const float* q, int D, int D_pad, const float* W, int nlist,
                         const float* bvec, double* xr) {
    const int ldw = nlist + D_pad;
    for (int j = 0; j < D_pad; ++j) {
        double acc = 0.0;
        for (int d = 0; d < D; ++d) acc = fma((double)q[d], (double)W[(int64_t)d * ldw + nlist + j], acc);
        xr[j] = acc + (double)bvec[nlist + j];
    }
}

/* (key, id) strictly-less for 64-bit keys (acc_hat bits << 32 | original id). */
static inline void insert_key(uint64_t* lk, int64_t* li, int K, uint64_t k, int64_t id) {
    if (!(k < lk[K - 1] || (k == lk[K - 1] && id < li[K - 1]))) return;
    int j = K - 1;
    while (j > 0 && (k < lk[j - 1] || (k == lk[j - 1] && id < li[j - 1]))) {
        lk[j] = lk[j - 1];
        li[j] = li[j - 1];
        --j;
    }
    lk[j] = k;
    li[j] = id;
}

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Modes 0 / 1.  Probe p of a query belongs to pass 1 when p < p_init and keeps k_p1 entries per
 * pair, else k_p2.  M > 0: rerank the pool's M best exactly (out_d = float32 of the float64
 * distance); M == 0: top-K by acc_hat (out_d = acc_hat).  Ids are original ids. */
int oracle_ivf_sq8(const float* xq, int64_t B, int D, int D_pad, const float* W, const float* bvec,
                   int nlist, const int32_t* probe_cids, int nprobe, int p_init,
                   const int32_t* vec_off, const int32_t* tile_off, int T,
                   const uint32_t* sq8_packed, const int32_t* tile_oids, const float* vmin,
                   const float* delta, int per_cluster, const float* xb_sorted, int K, int k_p1,
                   int k_p2, int M, float* out_d, int64_t* out_i, int nthreads) {
    if (K < 1 || D < 1 || D_pad < D || D_pad % 4 || k_p1 < 1 || k_p2 < 1 || M < 0) return -1;
    const int D4 = D_pad / 4;
    const int KL = M > 0 ? (M > K ? M : K) : K; /* pooled list length */
    int kmax = k_p1 > k_p2 ? k_p1 : k_p2;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        double* xr = (double*)malloc(sizeof(double) * (size_t)D_pad);
        float* base = (float*)malloc(sizeof(float) * (size_t)D_pad);
        uint64_t* pk = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)kmax);
        int64_t* pi = (int64_t*)malloc(sizeof(int64_t) * (size_t)kmax);
        uint64_t* gk = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)KL);
        int64_t* gi = (int64_t*)malloc(sizeof(int64_t) * (size_t)KL); /* sorted position */
        double* ld = (double*)malloc(sizeof(double) * (size_t)K);
        int64_t* li = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t q = 0; q < B; ++q) {
            const float* qv = xq + q * (int64_t)D;
            oracle_rotate_query(qv, D, D_pad, W, nlist, bvec, xr);
            for (int j = 0; j < KL; ++j) { gk[j] = UINT64_MAX; gi[j] = INT64_MAX; }
            for (int p = 0; p < nprobe; ++p) {
                const int32_t c = probe_cids[q * nprobe + p];
                if (c < 0) continue;
                const int kp = p < p_init ? k_p1 : k_p2;
                const int64_t off = per_cluster ? (int64_t)c * D_pad : 0;
                for (int d = 0; d < D_pad; ++d) base[d] = (float)((double)vmin[off + d] - xr[d]);
                for (int j = 0; j < kp; ++j) { pk[j] = UINT64_MAX; pi[j] = INT64_MAX; }
                const int64_t v0 = vec_off[c], n = vec_off[c + 1] - v0, t0 = tile_off[c];
                for (int64_t l = 0; l < n; ++l) {
                    const int64_t tile = t0 + l / T, slot = l % T;
                    float acc = 0.0f;
                    for (int d4 = 0; d4 < D4; ++d4) {
                        const uint32_t w = sq8_packed[(tile * D4 + d4) * T + slot];
                        for (int b = 0; b < 4; ++b) {
                            const int d = 4 * d4 + b;
                            const float a = fmaf((float)((w >> (8 * b)) & 0xffu), delta[off + d], base[d]);
                            acc = fmaf(a, a, acc);
                        }
                    }
                    const int32_t oid = tile_oids[tile * T + slot];
                    insert_key(pk, pi, kp, ((uint64_t)f32_bits(acc) << 32) | (uint32_t)oid, v0 + l);
                }
                for (int j = 0; j < kp && pk[j] != UINT64_MAX; ++j) insert_key(gk, gi, KL, pk[j], pi[j]);
            }
            if (M > 0) {
                for (int j = 0; j < K; ++j) { ld[j] = INFINITY; li[j] = INT64_MAX; }
                const int m = M < KL ? M : KL;
                for (int j = 0; j < m && gk[j] != UINT64_MAX; ++j) {
                    const double d = oracle_dist_f64(xb_sorted + gi[j] * D, qv, D);
                    insert_sorted(ld, li, K, d, (int64_t)(uint32_t)gk[j]);
                }
                for (int j = 0; j < K; ++j) {
                    const int valid = li[j] != INT64_MAX;
                    out_d[q * K + j] = valid ? (float)ld[j] : INFINITY;
                    out_i[q * K + j] = valid ? li[j] : -1;
                }
            } else {
                for (int j = 0; j < K; ++j) {
                    const int valid = gk[j] != UINT64_MAX;
                    out_d[q * K + j] = valid ? bits_f32((uint32_t)(gk[j] >> 32)) : INFINITY;
                    out_i[q * K + j] = valid ? (int64_t)(uint32_t)gk[j] : -1;
                }
            }
        }
        free(xr); free(base); free(pk); free(pi); free(gk); free(gi); free(ld); free(li);
    }
    return 0;
}

/* oracle_ivf_exact computed cluster-major, for large batches: the (query, probe) pairs are
 * grouped by cluster; each cluster's rows are read once, in chunks of 256 rows (kept in the
 * core's cache), for every query that probes it, into one top-K list per pair (by (d, id));
 * then each query merges its nprobe lists.  A row belongs to one list, so the merged list is
 * the top-K by (d, id) over the probed lists: the same result as oracle_ivf_exact (the same
 * canonical distances, the same order), with far fewer memory reads when many queries share
 * clusters.  Returns -2 when the pair lists or a thread's buffers cannot be allocated. */
int oracle_ivf_exact_cm(const float* xq, int64_t B, int D, const int32_t* probe_cids, int nprobe,
                        const int32_t* vec_off, const float* xb_sorted, const int32_t* orig_ids,
                        int nlist, int K, double* out_d, int64_t* out_i, int nthreads) {
    if (K < 1 || D < 1 || nlist < 1) return -1;
    const int64_t M = B * (int64_t)nprobe;
    int64_t* start = (int64_t*)calloc((size_t)nlist + 1, sizeof(int64_t));
    int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * (size_t)(M > 0 ? M : 1));
    double* pd = (double*)malloc(sizeof(double) * (size_t)(M > 0 ? M : 1) * (size_t)K);
    int64_t* pid = (int64_t*)malloc(sizeof(int64_t) * (size_t)(M > 0 ? M : 1) * (size_t)K);
    if (!start || !pairs || !pd || !pid) {
        free(start); free(pairs); free(pd); free(pid);
        return -2;
    }
    for (int64_t e = 0; e < M; ++e) {
        const int32_t c = probe_cids[e];
        if (c >= 0 && c < nlist) ++start[c + 1];
    }
    for (int c = 0; c < nlist; ++c) start[c + 1] += start[c];
    {
        int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (size_t)nlist);
        if (!fill) { free(start); free(pairs); free(pd); free(pid); return -2; }
        memcpy(fill, start, sizeof(int64_t) * (size_t)nlist);
        for (int64_t e = 0; e < M; ++e) {
            const int32_t c = probe_cids[e];
            if (c >= 0 && c < nlist) pairs[fill[c]++] = e; /* e = q * nprobe + p */
        }
        free(fill);
    }
    for (int64_t e = 0; e < M * K; ++e) { pd[e] = INFINITY; pid[e] = INT64_MAX; }
    /* Each chunk of CH rows is copied once per cluster, as float64 and dimension-major
     * (xt[d * CH + r] = (double)x_r,d), so that 32 rows' fma chains run side by side in
     * contiguous vectors; every row still gets t = (double)x_d - (double)q_d and
     * acc = fma(t, t, acc) for d in order, so the distances are oracle_dist_f64's. */
    const int CH = D <= 256 ? 256 : 64;
    int bad_alloc = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        double* xt = (double*)malloc(sizeof(double) * (size_t)CH * (size_t)D);
        double* q64 = (double*)malloc(sizeof(double) * (size_t)D);
        double* dd = (double*)malloc(sizeof(double) * (size_t)CH);
        if (!xt || !q64 || !dd) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            bad_alloc = 1;
        }
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int c = 0; c < nlist; ++c) {
            if (!xt || !q64 || !dd) continue;
            const int64_t v0 = vec_off[c], v1 = vec_off[c + 1];
            for (int64_t cb = v0; cb < v1 && start[c + 1] > start[c]; cb += CH) {
                const int n = (int)((cb + CH < v1 ? cb + CH : v1) - cb);
                const int n32 = (n + 31) & ~31;
                for (int r = 0; r < n32; ++r)
                    for (int d = 0; d < D; ++d)
                        xt[(int64_t)d * CH + r] = r < n ? (double)xb_sorted[(cb + r) * D + d] : 0.0;
                for (int64_t k = start[c]; k < start[c + 1]; ++k) {
                    const int64_t e = pairs[k];
                    const float* qv = xq + (e / nprobe) * (int64_t)D;
                    for (int d = 0; d < D; ++d) q64[d] = (double)qv[d];
                    for (int g = 0; g < n32; g += 32) {
                        double a[32];
                        for (int r = 0; r < 32; ++r) a[r] = 0.0;
                        for (int d = 0; d < D; ++d) {
                            const double qd = q64[d];
                            const double* xr = xt + (int64_t)d * CH + g;
                            for (int r = 0; r < 32; ++r) {
                                const double t = xr[r] - qd;
                                a[r] = fma(t, t, a[r]);
                            }
                        }
                        for (int r = 0; r < 32; ++r) dd[g + r] = a[r];
                    }
                    double* ld = pd + e * K;
                    int64_t* li = pid + e * K;
                    for (int r = 0; r < n; ++r) insert_sorted(ld, li, K, dd[r], (int64_t)orig_ids[cb + r]);
                }
            }
        }
        free(xt);
        free(q64);
        free(dd);
    }
    if (bad_alloc) {
        free(start); free(pairs); free(pd); free(pid);
        return -2;
    }
#ifdef _OPENMP
#pragma omp parallel
#endif
    {
        double* ld = (double*)malloc(sizeof(double) * (size_t)K);
        int64_t* li = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t q = 0; q < B; ++q) {
            for (int j = 0; j < K; ++j) { ld[j] = INFINITY; li[j] = INT64_MAX; }
            for (int64_t e = q * nprobe; e < (q + 1) * nprobe; ++e)
                for (int j = 0; j < K && pid[e * K + j] != INT64_MAX; ++j)
                    insert_sorted(ld, li, K, pd[e * K + j], pid[e * K + j]);
            for (int j = 0; j < K; ++j) {
                const int valid = li[j] != INT64_MAX;
                out_d[q * K + j] = valid ? ld[j] : INFINITY;
                out_i[q * K + j] = valid ? li[j] : -1;
            }
        }
        free(ld);
        free(li);
    }
    free(start); free(pairs); free(pd); free(pid);
    return 0;
}

/* Canonical float64 distances for an explicit list of (query, sorted-position) pairs. */
int oracle_pair_dists(const float* xq, int D, const float* xb_sorted, const int32_t* qids,
                      const int64_t* spos, int64_t n, double* out_d) {
    for (int64_t i = 0; i < n; ++i)
        out_d[i] = oracle_dist_f64(xb_sorted + spos[i] * D, xq + (int64_t)qids[i] * D, D);
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
