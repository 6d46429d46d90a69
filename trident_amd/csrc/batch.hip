// Cluster-batched cascade on the gfx950 int8 matrix cores.
//
// When many queries probe the same cluster (r = B * nprobe / nlist is ~600 at cfg 2), the SQ8
// bound is a dense contraction: codes [n_c x D_pad] (u8) times per-query weights
// [D_pad x queries].  For vector x (codes c_d, cluster vmin/delta) and query q with
// q'_d = q_rot,d - vmin_d and w_d = delta_d * q'_d:
//
//     |x_hat - q_rot|^2 = A_x - 2 sum_d c_d w_d + Q_q,   A_x = sum_d (c_d delta_d)^2,  Q_q = |q'|^2
//
// w is quantised per query to w = s * w_int + err (s a power of two, |w_int| <= 32639, split
// w_int = 256 * hi + lo into two int8 planes); with c' = c - 128 the dot product
//     sum_d c_d w_int,d = 256 * MFMA(c', hi) + MFMA(c', lo) + 128 * sum_d w_int,d
// is computed EXACTLY by v_mfma_i32_16x16x64_i8 (two per 64 dims), and
// |sum_d c_d w_d - s * dot| <= 255 * sum_d |w_d - s w_int,d| = err_q.  The triangle inequality
// with r_x >= |x_rot - x_hat| (per vector) and e_q >= |q_rot(float64) - q_rot(exact)| gives
//     lower bound:  |x_rot - q_rot| >= sqrt(A_x + Q_q - 2 s dot - 2 err_q) - r_x - e_q
//     upper bound:  |x_rot - q_rot| <= sqrt(A_x + Q_q - 2 s dot + 2 err_q) + r_x + e_q
// (this norm form keeps the per-dimension bound's selectivity: the same 0.006% survivors on
// cfg-2 data).  Scaled by the rotation's squared singular-value bounds these bound the
// canonical float64 distance.
//
// Pass A (UB):  for the first p_init probes of each query, the K-th smallest upper bound over
//               the cluster -> atomicMin into tau[q] (the reference's Stage X seeding,
//               src/trident_v4_kernels.cu:626-676, computed for a block of queries at once).
// Pass B (LB):  for every probe, lanes whose lower bound passes tau[q] are compacted into a
//               per-wave queue and refined exactly in float64 (canonical order); distances
//               <= tau[q] are appended to the query's candidate list.
//
// One workgroup per (cluster, block of <= 64 pairs); its 4 waves are independent and own 16
// queries each (the MFMA N dimension).  Lane l = (i = l & 15, g = l >> 4) holds, for every
// 64-dim step, bytes of dims step*64 + g*16 + [0, 16): vector i's codes in the A operand and
// query i's weights in the B operand (any dim-to-byte assignment shared by A and B computes
// the same contraction); the result row 4g + r, column i sits in lane l, register r.
#include "common.hpp"
#include "kernels.hpp"

namespace trident {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kQW = 16;                          // queries per wave
constexpr int kChunkQ = kQW * kWavesPerBlock;    // pairs per workgroup chunk
constexpr int kMaxKS = 4;                        // 64-dim steps held in registers (D_pad <= 256)
constexpr int kUbList = 16;                      // per-lane upper-bound list (K <= 64)
constexpr int kBStageCh = 32;
constexpr int kBQueue = 128;

// grid 2 (one block per pass): chunk table of the pass's cluster segments.
__global__ __launch_bounds__(256) void build_chunks_kernel(const int32_t* seg_off, int nlist,
                                                           int32_t* chunk_cid, int32_t* chunk_start,
                                                           int32_t* chunk_cnt, int32_t* n_chunks,
                                                           int max_chunks) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int pass = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int32_t* off = seg_off + pass * (nlist + 1);
    int32_t* cc = chunk_cid + pass * max_chunks;
    int32_t* cs = chunk_start + pass * max_chunks;
    int32_t* cn = chunk_cnt + pass * max_chunks;
    const int per = (nlist + kBlock - 1) / kBlock;
    const int c0 = min(nlist, tid * per), c1 = min(nlist, c0 + per);
    uint32_t local = 0;
    for (int c = c0; c < c1; ++c) local += (uint32_t)((off[c + 1] - off[c] + kChunkQ - 1) / kChunkQ);
    uint32_t inc = local;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        uint32_t t = (uint32_t)__shfl_up((int)inc, o, kWave);
        if (lane >= o) inc += t;
    }
    if (lane == kWave - 1) s_wtot[wid] = inc;
    __syncthreads();
    uint32_t run = inc - local, total = 0;
    for (int w = 0; w < kWavesPerBlock; ++w) {
        if (w < wid) run += s_wtot[w];
        total += s_wtot[w];
    }
    for (int c = c0; c < c1; ++c) {
        for (int s = off[c]; s < off[c + 1]; s += kChunkQ) {
            if ((int)run < max_chunks) {
                cc[run] = c;
                cs[run] = s;
                cn[run] = min(kChunkQ, off[c + 1] - s);
            }
            ++run;
        }
    }
    if (tid == 0) n_chunks[pass] = (int32_t)min<uint32_t>(total, (uint32_t)max_chunks);
}

__global__ void fill_u64_kernel(unsigned long long* p, unsigned long long v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__device__ __forceinline__ double shfl_f64(double v, int src) {
    const uint64_t k = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)k, src, kWave);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(k >> 32), src, kWave);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Canonical float64 distance of queued survivors; lane s < cnt refines survivor s against its
// own query row (float32 queries, widened exactly).  Base rows are staged through LDS with
// 128-byte coalesced loads (the same pattern serves mapped host memory).
__device__ __forceinline__ double refine_multi(const float* __restrict__ xb,
                                               const float* __restrict__ xq, int D,
                                               const int32_t* spos_of, int cnt, int my_q,
                                               float (*stage)[kWave + 1]) {
    const int lane = lane_id();
    const int half = lane >> 5, kk = lane & 31;
    double acc = 0.0;
    const float* qrow = xq + (size_t)my_q * D;
    for (int d0 = 0; d0 < D; d0 += kBStageCh) {
        const int ch = min(kBStageCh, D - d0);
        for (int r0 = 0; r0 < cnt; r0 += 2) {
            const int r = r0 + half;
            float v = 0.0f;
            if (r < cnt && kk < ch) v = xb[(size_t)spos_of[r] * D + d0 + kk];
            if (r < cnt) stage[kk][r] = v;
        }
        wave_sync();
        if (lane < cnt) {
            for (int k = 0; k < ch; ++k) {
                const double t = (double)stage[k][lane] - (double)qrow[d0 + k];
                acc = fma(t, t, acc);
            }
        }
        wave_sync();
    }
    return acc;
}

template <bool UB_PASS>
__global__ __launch_bounds__(256) void batch_scan_kernel(BatchArgs a) {
    __shared__ float s_stage[kWavesPerBlock][kBStageCh][kWave + 1];
    __shared__ int32_t s_queue[kWavesPerBlock][kBQueue];
    __shared__ int32_t s_spos[kWavesPerBlock][kWave];

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int total = a.n_chunks[0];
    const int nx = (total + 7) >> 3;
    const int ch = (int)(blockIdx.x & 7) * nx + (int)(blockIdx.x >> 3);
    if ((int)(blockIdx.x >> 3) >= nx || ch >= total) return;
    const int cid = a.chunk_cid[ch], start = a.chunk_start[ch], cnt = a.chunk_cnt[ch];
    const int qb = wid * kQW;
    if (qb >= cnt) return;
    const int nq = min(kQW, cnt - qb);
    const int j = lane & 15, g = lane >> 4;
    const bool hasq = j < nq;
    const int q = a.pair_qid[start + qb + (hasq ? j : 0)];
    const int v0 = a.vec_off[cid], n = a.vec_off[cid + 1] - v0;
    if (n <= 0) return;
    const int t0 = a.tile_off[cid];
    const int D_pad = a.D_pad, D4 = D_pad >> 2, T = a.T;
    const int KS = (D_pad + 63) >> 6;
    const size_t off = a.per_cluster ? (size_t)cid * D_pad : 0;
    const double* xr = a.xrot64 + (size_t)q * D_pad;
    const double* qe = a.qerr + (size_t)q * D_pad;

    // ---- per-query weights for this lane's dims ----
    double mx = 0.0, Qp = 0.0, ep = 0.0;
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll 4
        for (int t = 0; t < 16; ++t) {
            const int d = ks * 64 + g * 16 + t;
            if (d < D_pad) {
                const double qp = xr[d] - (double)a.vmin[off + d];
                const double w = (double)a.delta[off + d] * qp;
                mx = fmax(mx, fabs(w));
                Qp = fma(qp, qp, Qp);
                ep = fma(qe[d], qe[d], ep);
            }
        }
    }
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
        mx = fmax(mx, shfl_f64(mx, lane ^ o));
        Qp += shfl_f64(Qp, lane ^ o);
        ep += shfl_f64(ep, lane ^ o);
    }
    double s = 1.0;
    if (mx > 0.0) {
        s = ldexp(1.0, ilogb(mx) - 14);
        if (mx / s > 32639.0) s *= 2.0;
    }
    v4i bhi[kMaxKS], blo[kMaxKS];
    double errs = 0.0;
    int wsum = 0;
#pragma unroll
    for (int ks = 0; ks < kMaxKS; ++ks) {
        uint32_t hw[4] = {0u, 0u, 0u, 0u}, lw[4] = {0u, 0u, 0u, 0u};
        if (ks < KS) {
            for (int t = 0; t < 16; ++t) {
                const int d = ks * 64 + g * 16 + t;
                int wi = 0;
                if (d < D_pad) {
                    const double qp = xr[d] - (double)a.vmin[off + d];
                    const double w = (double)a.delta[off + d] * qp;
                    wi = (int)rint(w / s);
                    errs += fabs(w - s * (double)wi) + 0x1p-52 * fabs(w);
                }
                const int hi = (wi + 128) >> 8;
                const int lo = wi - (hi << 8);
                wsum += wi;
                hw[t >> 2] |= ((uint32_t)hi & 0xffu) << (8 * (t & 3));
                lw[t >> 2] |= ((uint32_t)lo & 0xffu) << (8 * (t & 3));
            }
        }
        bhi[ks] = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
        blo[ks] = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
    }
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
        errs += shfl_f64(errs, lane ^ o);
        wsum += __shfl_xor(wsum, o, kWave);
    }
    const double err_q = 255.0 * errs * (1.0 + 0x1p-40);
    const double e_q = sqrt(ep) * (1.0 + 1e-12) + 0x1p-52 * sqrt(Qp) + 1e-300;
    const double cW = 128.0 * (double)wsum;
    const double c1 = 2.0 * s;

    // thresholds
    double tau = (double)INFINITY;
    double G = 0.0, c2 = 0.0, AQ = 0.0;
    bool pass_all = true;
    if constexpr (UB_PASS) {
        AQ = (Qp + 2.0 * err_q) * (1.0 + 1e-13);
    } else {
        tau = a.tau[q];
        if (tau < (double)INFINITY) {
            pass_all = false;
            const double tq = sqrt(tau * a.rot_sq_max) * (1.0 + 1e-12) + e_q;
            G = 2.0 * err_q - Qp * (1.0 - 1e-13) + tq * tq;
            c2 = -2.0 * tq;
        }
    }

    float ubl[kUbList];
    if constexpr (UB_PASS) {
#pragma unroll
        for (int i = 0; i < kUbList; ++i) ubl[i] = INFINITY;
    }
    int qn = 0;
    unsigned long long st_cand = 0, st_surv = 0, st_ins = 0;
    int32_t* my_queue = s_queue[wid];
    int32_t* my_spos = s_spos[wid];
    float(*my_stage)[kWave + 1] = s_stage[wid];

    auto flush = [&](int fcnt) {
        int e = 0, my_sq = q;
        double my_tau = tau;
        if (lane < fcnt) e = my_queue[lane];
        const int li = e >> 4, jj = e & 15;
        my_sq = __shfl(q, jj, kWave);
        my_tau = shfl_f64(tau, jj);
        if (lane < fcnt) my_spos[lane] = v0 + li;
        wave_sync();
        const double d64 = refine_multi(a.xb, a.xq, a.D, my_spos, fcnt, my_sq, my_stage);
        const bool ok = lane < fcnt && d64 <= my_tau;
        if (a.stats) st_ins += __popcll(__ballot(ok));
        if (ok) {
            const int slot = atomicAdd(&a.cand_cnt[my_sq], 1);
            if (slot < a.cap) {
                a.cand_key[(size_t)my_sq * a.cap + slot] = key_of(d64);
                a.cand_id[(size_t)my_sq * a.cap + slot] = a.tile_oids[(size_t)t0 * T + li];
            }
        }
        wave_sync();
    };

    const int ntl = (n + 15) >> 4;
    for (int tt = 0; tt < ntl; ++tt) {
        // A operand: codes of vector tt*16 + (lane & 15), dims ks*64 + g*16 + [0, 16)
        const int lia = tt * 16 + j;
        const bool va = lia < n;
        const uint32_t* cp = a.sq8 + ((size_t)(t0 + lia / T) * D4) * T + (lia % T);
        v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < kMaxKS; ++ks) {
            if (ks < KS) {
                v4i av;
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4) {
                    const int d4 = ks * 16 + g * 4 + t4;
                    const uint32_t wv = (va && d4 < D4) ? cp[(size_t)d4 * T] : 0x80808080u;
                    av[t4] = (int)(wv ^ 0x80808080u);
                }
                acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bhi[ks], acc_hi, 0, 0, 0);
                acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, blo[ks], acc_lo, 0, 0, 0);
            }
        }
        // epilogue: rows 4g + r (vectors), column j (query)
        uint32_t sbits = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int li = tt * 16 + 4 * g + r;
            const bool ok = hasq && li < n;
            const double dot = (double)((acc_hi[r] << 8) + acc_lo[r]) + cW;
            const double2 ar = ok ? *reinterpret_cast<const double2*>(a.vec_Ar + 2 * (size_t)(v0 + li))
                                  : double2{0.0, 0.0};
            if constexpr (UB_PASS) {
                if (ok) {
                    const double E = fmax(fma(-c1, dot, ar.x * (1.0 + 1e-13) + AQ), 0.0);
                    const float s32 = sqrtf((float)(E * (1.0 + 1e-12))) * (1.0f + 0x1p-20f);
                    const float u = (s32 + (float)ar.y + (float)e_q) * (1.0f + 0x1p-20f);
                    if (u < ubl[kUbList - 1]) {
#pragma unroll
                        for (int i = kUbList - 1; i > 0; --i)
                            ubl[i] = (u < ubl[i - 1]) ? ubl[i - 1] : fminf(ubl[i], u);
                        ubl[0] = fminf(ubl[0], u);
                    }
                }
            } else {
                bool sv = ok;
                if (ok && !pass_all) {
                    const double lhs = fma(c2, ar.y, fma(-ar.y, ar.y, ar.x * (1.0 - 1e-13)));
                    const double rhs = fma(c1, dot, G);
                    sv = lhs <= rhs;
                }
                sbits |= (uint32_t)sv << r;
            }
        }
        if (a.stats) st_cand += (unsigned long long)nq * (unsigned long long)min(16, n - tt * 16);
        if constexpr (!UB_PASS) {
            if (__ballot(sbits != 0) == 0) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool sv = (sbits >> r) & 1u;
                const uint64_t m = __ballot(sv);
                if (m == 0) continue;
                if (sv) my_queue[qn + mask_rank(m)] = ((tt * 16 + 4 * g + r) << 4) | j;
                qn += __popcll(m);
                if (a.stats) st_surv += __popcll(m);
                if (qn >= kWave) {
                    wave_sync();
                    flush(kWave);
                    const int rest = qn - kWave;
                    int32_t keep = 0;
                    if (lane < rest) keep = my_queue[kWave + lane];
                    wave_sync();
                    if (lane < rest) my_queue[lane] = keep;
                    qn = rest;
                    wave_sync();
                }
            }
        }
    }

    if constexpr (UB_PASS) {
        // K-th smallest upper bound of each query: merge the 4 lanes' lists (64 values) by a
        // register bitonic sort, then atomicMin into tau[q] (float64 bit pattern).
        float* s_ub = &my_stage[0][0];
#pragma unroll
        for (int i = 0; i < kUbList; ++i) s_ub[j * 64 + g * kUbList + i] = ubl[i];
        wave_sync();
        for (int jj = 0; jj < nq; ++jj) {
            uint64_t k = key_of((double)s_ub[jj * 64 + lane]);
            int32_t id = lane;
            wave_sort64(k, id);
            const uint64_t kk = readlane_u64(k, a.K - 1);
            const int qq = __shfl(q, jj, kWave);
            if (lane == 0 && dist_of(kk) < (double)INFINITY) {
                const double u = dist_of(kk);
                const double tub = u * u / a.rot_sq_min * (1.0 + 1e-6);
                atomicMin(reinterpret_cast<unsigned long long*>(a.tau) + qq,
                          (unsigned long long)key_of(tub));
            }
        }
    } else if (qn > 0) {
        wave_sync();
        flush(qn);
    }
    if (a.stats && lane == 0) {
        const int slot = (int)(blockIdx.x % kStatSlots) * 4;
        atomicAdd(&a.stats[slot + 0], st_cand);
        atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)D_pad);
        atomicAdd(&a.stats[slot + 2], st_surv);
        atomicAdd(&a.stats[slot + 3], st_ins);
    }
}

template __global__ void batch_scan_kernel<true>(BatchArgs);
template __global__ void batch_scan_kernel<false>(BatchArgs);

}  // namespace trident

namespace trident {

// tau_sq output of the batched route: the seeded float64 threshold, rounded up to float32.
__global__ void tau_to_f32_kernel(const double* tau, float* out, int B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) out[i] = __double2float_ru(tau[i]);
}

}  // namespace trident
