// Front end of the lossless IVF query path on gfx950: query preparation (float64 copy,
// float64 PCA rotation with a rigorous error bound), float64 coarse distances, the exact
// (d, cid) top-nprobe selection, and the cluster-major grouping of (cluster, query) pairs.
//
// Reference counterparts (src/trident_v4_kernels.cu): the fused coarse+rotation GEMM
// at::addmm_out (:1233-1246), trident_topk_centroids_kernel (:68-162) and
// trident_counting_sort_pairs_kernel (:168-263).  The reference forms coarse distances as
// |c|^2 - 2<q,c> + |q|^2 in FP32, which can reorder near-tied centroids; here every
// (query, centroid) distance is the canonical float64 sum of squared differences in
// dimension order, so the probe set equals the float64 oracle's on every query.
#include "common.hpp"
#include "kernels.hpp"

namespace trident {

__global__ void fill_i32_kernel(int32_t* p, int32_t v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// grid (ceil(max(D, D_pad) / 64), ceil(B / (4 kPrepQB))), block (64, 4): each wave takes
// kPrepQB queries (wave-uniform rows, scalar loads) x 64 columns, so every loaded rotation value
// feeds kPrepQB chains.
// xq64[b, d] = (double)xq[b, d]; xrot64[b, j] = sum_d xq[b, d] * R[d, j] + bvec[j] evaluated
// in float64 (fma, dimension order), xrot32 = xrot64 rounded to float32, and qerr[b, j] bounds
// the distance of xrot64 from the exact value.
__global__ __launch_bounds__(256) void prep_queries_kernel(
    const float* __restrict__ xq, int B, int D, int D_pad, const float* __restrict__ W, int ldw,
    int nlist, const float* __restrict__ bvec, double* __restrict__ xq64,
    double* __restrict__ xrot64, float* __restrict__ xrot32, double* __restrict__ qerr,
    int do_rot) {
    constexpr int QB = kPrepQB;
    const int j = blockIdx.x * 64 + threadIdx.x;
    const int b0 = (blockIdx.y * 4 + threadIdx.y) * QB;
    if (b0 >= B) return;
    const float* qr[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) qr[i] = xq + (size_t)min(b0 + i, B - 1) * D;
    if (j < D) {
#pragma unroll
        for (int i = 0; i < QB; ++i)
            if (b0 + i < B) xq64[(size_t)(b0 + i) * D + j] = (double)qr[i][j];
    }
    if (!do_rot || j >= D_pad) return;
    double acc[QB], mag[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) acc[i] = mag[i] = 0.0;
    const float* wcol = W + nlist + j;
#pragma unroll 4
    for (int d = 0; d < D; ++d) {
        const double r = (double)wcol[(size_t)d * ldw];
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            const double qd = (double)qr[i][d];
            acc[i] = fma(qd, r, acc[i]);
            mag[i] += fabs(qd * r);
        }
    }
    const double bj = (double)bvec[nlist + j];
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        if (b0 + i >= B) break;
        const double xr = acc[i] + bj;
        xrot64[(size_t)(b0 + i) * D_pad + j] = xr;
        xrot32[(size_t)(b0 + i) * D_pad + j] = (float)xr;
        // |fl(sum) - sum| <= (D + 1) 2^-53 sum|terms|; doubled to also cover the rounding of
        // `mag`.
        qerr[(size_t)(b0 + i) * D_pad + j] =
            (double)(D + 3) * 0x1p-52 * (mag[i] + fabs(bj)) + 0x1p-1000;
    }
}

// grid (ceil(nlist / (64 kCoarseNC)), ceil(B / (kCoarseQW * 4))), block 256: each wave owns
// kCoarseQW queries x 64 kCoarseNC centroids, each lane kCoarseNC centroids (c = base + lane +
// 64 k) x kCoarseQW queries in registers.  Query values are wave-uniform (scalar loads, two
// dims at a time when the rows allow it), so every loaded value feeds kCoarseNC (queries) or
// kCoarseQW (centroids) fma chains.  Centroid c, dim d is -0.5f * W[d, c], exact because
// W_coarse_only = -2 C^T.  Each (query, centroid) sum is one fma chain in dimension order:
// t = q_d - c_d, acc = fma(t, t, acc).
__global__ __launch_bounds__(256) void coarse_dist_kernel(const double* __restrict__ xq64, int B,
                                                          int D, const float* __restrict__ W,
                                                          int ldw, int nlist,
                                                          double* __restrict__ cd64) {
    constexpr int QW = kCoarseQW, NC = kCoarseNC;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c0 = blockIdx.x * (64 * NC) + lane;
    const int qb = blockIdx.y * (QW * kWavesPerBlock) + wid * QW;
    if (qb >= B) return;
    const double* qrow[QW];
#pragma unroll
    for (int i = 0; i < QW; ++i) qrow[i] = xq64 + (size_t)min(qb + i, B - 1) * D;
    const float* wc[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) wc[k] = W + min(c0 + 64 * k, nlist - 1);
    double acc[QW][NC];
#pragma unroll
    for (int i = 0; i < QW; ++i)
#pragma unroll
        for (int k = 0; k < NC; ++k) acc[i][k] = 0.0;
    int d = 0;
    if ((D & 1) == 0) {  // rows are 16-byte aligned: xq64 is 256-byte aligned, D even
        for (; d < D; d += 2) {
            double cv0[NC], cv1[NC];
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                cv0[k] = (double)(-0.5f * wc[k][(size_t)d * ldw]);
                cv1[k] = (double)(-0.5f * wc[k][(size_t)(d + 1) * ldw]);
            }
#pragma unroll
            for (int i = 0; i < QW; ++i) {
                const double2 qv = *reinterpret_cast<const double2*>(qrow[i] + d);
#pragma unroll
                for (int k = 0; k < NC; ++k) {
                    double t = qv.x - cv0[k];
                    acc[i][k] = fma(t, t, acc[i][k]);
                    t = qv.y - cv1[k];
                    acc[i][k] = fma(t, t, acc[i][k]);
                }
            }
        }
    }
    for (; d < D; ++d) {
        double cv[NC];
#pragma unroll
        for (int k = 0; k < NC; ++k) cv[k] = (double)(-0.5f * wc[k][(size_t)d * ldw]);
#pragma unroll
        for (int i = 0; i < QW; ++i) {
            const double qv = qrow[i][d];
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                const double t = qv - cv[k];
                acc[i][k] = fma(t, t, acc[i][k]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int c = c0 + 64 * k;
        if (c < nlist) {
#pragma unroll
            for (int i = 0; i < QW; ++i)
                if (qb + i < B) cd64[(size_t)(qb + i) * nlist + c] = acc[i][k];
        }
    }
}

// Block-wide exclusive scan of one uint32 per thread (256 threads).
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave_tot,
                                                         uint32_t* total) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        uint32_t t = (uint32_t)__shfl_up((int)inc, o, kWave);
        if (lane >= o) inc += t;
    }
    if (lane == kWave - 1) s_wave_tot[wid] = inc;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
        const uint32_t t = s_wave_tot[w];
        if (w < wid) before += t;
        all += t;
    }
    __syncthreads();
    if (total) *total = all;
    return before + inc - v;
}

// One block of 256 threads per query.  Radix-selects the exact nprobe-th smallest float64
// key, takes every smaller key plus the smallest cids among the equal ones, then sorts the
// selection by (d, cid).  Keys live in LDS (nlist * 8 bytes of dynamic LDS).  Results go to
// out_* (stride ld) and, when non-null, are mirrored into out2_* (stride ld2).
__global__ __launch_bounds__(256) void select_probes_kernel(const double* __restrict__ cd64,
                                                            int nlist, int nprobe,
                                                            int32_t* __restrict__ out_cids,
                                                            float* __restrict__ out_dqcs, int ld,
                                                            int32_t* __restrict__ out2_cids,
                                                            float* __restrict__ out2_dqcs,
                                                            int ld2) {
    extern __shared__ uint64_t s_keys[];
    __shared__ uint32_t s_hist[256];
    __shared__ uint64_t s_sel_k[512];
    __shared__ int32_t s_sel_c[512];
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    __shared__ uint64_t s_red[2][kWavesPerBlock];
    __shared__ uint32_t s_digit, s_need, s_nsel;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int q = blockIdx.x;
    const double* row = cd64 + (size_t)q * nlist;

    uint64_t kmin = kKeyInvalid, kmax = 0;
    for (int c = tid; c < nlist; c += kBlock) {
        const uint64_t k = key_of(row[c]);
        s_keys[c] = k;
        kmin = k < kmin ? k : kmin;
        kmax = k > kmax ? k : kmax;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t a = shfl_xor_u64(kmin, o), b = shfl_xor_u64(kmax, o);
        kmin = a < kmin ? a : kmin;
        kmax = b > kmax ? b : kmax;
    }
    if (lane == 0) {
        s_red[0][wid] = kmin;
        s_red[1][wid] = kmax;
    }
    __syncthreads();
    kmin = s_red[0][0];
    kmax = s_red[1][0];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) {
        kmin = s_red[0][w] < kmin ? s_red[0][w] : kmin;
        kmax = s_red[1][w] > kmax ? s_red[1][w] : kmax;
    }

    // Radix select over the digits below the common prefix of all keys.
    uint64_t prefix = kmin, mask = ~0ull;
    uint32_t need = (uint32_t)nprobe;
    const uint64_t diff = kmin ^ kmax;
    if (diff != 0) {
        const int top = 63 - __clzll((long long)diff);
        const int start = (top >> 3) << 3;
        mask = (start + 8 >= 64) ? 0ull : (~0ull << (start + 8));
        prefix = kmin & mask;
        for (int shift = start; shift >= 0; shift -= 8) {
            s_hist[tid] = 0;
            __syncthreads();
            for (int c = tid; c < nlist; c += kBlock) {
                const uint64_t k = s_keys[c];
                if ((k & mask) == prefix) atomicAdd(&s_hist[(k >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (wid == 0) {
                uint32_t h[4];
                uint32_t loc = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    h[i] = s_hist[4 * lane + i];
                    loc += h[i];
                }
                uint32_t inc = loc;
#pragma unroll
                for (int o = 1; o < kWave; o <<= 1) {
                    uint32_t t = (uint32_t)__shfl_up((int)inc, o, kWave);
                    if (lane >= o) inc += t;
                }
                const uint32_t exc = inc - loc;
                if (exc < need && need <= inc) {
                    uint32_t cum = exc;
                    int bsel = 3;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (cum + h[i] >= need) {
                            bsel = i;
                            break;
                        }
                        cum += h[i];
                    }
                    s_digit = (uint32_t)(4 * lane + bsel);
                    s_need = need - cum;
                }
            }
            __syncthreads();
            prefix |= (uint64_t)s_digit << shift;
            mask |= 255ull << shift;
            need = s_need;
            __syncthreads();
        }
    }
    const uint64_t kstar = prefix;

    // Take all keys < kstar and the `need` smallest cids among keys == kstar.
    const int chunk = (nlist + kBlock - 1) / kBlock;
    const int c0 = min(nlist, tid * chunk), c1 = min(nlist, c0 + chunk);
    uint32_t my_eq = 0;
    for (int c = c0; c < c1; ++c) my_eq += s_keys[c] == kstar;
    uint32_t rank = block_exclusive_scan(my_eq, s_wtot, nullptr);
    if (tid == 0) s_nsel = 0;
    __syncthreads();
    for (int c = c0; c < c1; ++c) {
        const uint64_t k = s_keys[c];
        bool take = k < kstar;
        if (k == kstar) {
            take = rank < need;
            ++rank;
        }
        if (take) {
            const uint32_t slot = atomicAdd(&s_nsel, 1u);
            s_sel_k[slot] = k;
            s_sel_c[slot] = c;
        }
    }
    int P2 = 1;
    while (P2 < nprobe) P2 <<= 1;
    __syncthreads();
    for (int i = nprobe + tid; i < P2; i += kBlock) {
        s_sel_k[i] = kKeyInvalid;
        s_sel_c[i] = kIdInvalid;
    }
    __syncthreads();
    for (int s = 2; s <= P2; s <<= 1) {
        for (int j = s >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < (P2 >> 1); i += kBlock) {
                const int lo = 2 * j * (i / j) + (i % j), hi = lo + j;
                const bool up = (lo & s) == 0;
                const uint64_t kl = s_sel_k[lo], kh = s_sel_k[hi];
                const int32_t cl = s_sel_c[lo], ch = s_sel_c[hi];
                const bool hi_less = ent_less(kh, ch, kl, cl);
                if (hi_less == up) {
                    s_sel_k[lo] = kh;
                    s_sel_k[hi] = kl;
                    s_sel_c[lo] = ch;
                    s_sel_c[hi] = cl;
                }
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < nprobe; i += kBlock) {
        const int32_t c = s_sel_c[i];
        const float dq = (float)sqrt(dist_of(s_sel_k[i]));
        out_cids[(size_t)q * ld + i] = c;
        out_dqcs[(size_t)q * ld + i] = dq;
        if (out2_cids) out2_cids[(size_t)q * ld2 + i] = c;
        if (out2_dqcs) out2_dqcs[(size_t)q * ld2 + i] = dq;
    }
}

// counts: [2, nlist + 1] (pass-1 row, pass-2 row), zeroed by the caller.
__global__ void count_pairs_kernel(const int32_t* __restrict__ probe_cids, int ld, int B,
                                   int nprobe, int p_init, int nlist, int32_t* counts) {
    const int64_t total = (int64_t)B * nprobe;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int q = (int)(idx / nprobe), p = (int)(idx - (int64_t)q * nprobe);
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;  // invalid caller input: never index
        atomicAdd(&counts[(p < p_init ? 0 : (nlist + 1)) + cid], 1);
    }
}

// grid 2 (one block per pass), block 256: seg_off[pass] = exclusive scan of counts[pass];
// cursor[pass] receives the same offsets for the scatter.
__global__ __launch_bounds__(256) void scan_pairs_kernel(const int32_t* counts, int nlist,
                                                         int32_t* seg_off, int32_t* cursor) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int pass = blockIdx.x, tid = threadIdx.x;
    const int32_t* cnt = counts + pass * (nlist + 1);
    int32_t* off = seg_off + pass * (nlist + 1);
    int32_t* cur = cursor + pass * (nlist + 1);
    const int chunk = (nlist + kBlock - 1) / kBlock;
    const int c0 = min(nlist, tid * chunk), c1 = min(nlist, c0 + chunk);
    uint32_t local = 0;
    for (int c = c0; c < c1; ++c) local += (uint32_t)cnt[c];
    uint32_t total = 0;
    uint32_t run = block_exclusive_scan(local, s_wtot, &total);
    for (int c = c0; c < c1; ++c) {
        const uint32_t v = (uint32_t)cnt[c];
        off[c] = (int32_t)run;
        cur[c] = (int32_t)run;
        run += v;
    }
    if (tid == 0) {
        off[nlist] = (int32_t)total;
        cur[nlist] = (int32_t)total;
    }
}

__global__ void scatter_pairs_kernel(const int32_t* __restrict__ probe_cids,
                                     const float* __restrict__ probe_dqcs, int ld, int B,
                                     int nprobe, int p_init, int nlist, int32_t* cursor,
                                     int32_t* __restrict__ p1_cids, int32_t* __restrict__ p1_qids,
                                     float* __restrict__ p1_dqcs, int32_t* __restrict__ p2_cids,
                                     int32_t* __restrict__ p2_qids, float* __restrict__ p2_dqcs) {
    const int64_t total = (int64_t)B * nprobe;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int q = (int)(idx / nprobe), p = (int)(idx - (int64_t)q * nprobe);
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;  // invalid caller input: never index
        const bool first = p < p_init;
        const int slot = atomicAdd(&cursor[(first ? 0 : (nlist + 1)) + cid], 1);
        int32_t* oc = first ? p1_cids : p2_cids;
        int32_t* oq = first ? p1_qids : p2_qids;
        float* od = first ? p1_dqcs : p2_dqcs;
        oc[slot] = cid;
        oq[slot] = q;
        if (od) od[slot] = probe_dqcs ? probe_dqcs[(size_t)q * ld + p] : 0.0f;
    }
}

// One wave per query (nprobe <= KP): the query's float64 centroid distances go through a
// register list of the KP best (d, cid) entries, sorted across lanes.  Each chunk of 1024 keys
// (16 per lane) is first cut at T0 = the largest over lanes of each lane's r-th smallest entry,
// r = ceil(nprobe / 64): at least nprobe entries are <= T0, so nothing above T0 (or above the
// list's current nprobe-th entry) can be selected.  The few entries below the cut are compacted
// through LDS and merged in batches of 64.  Same (d, cid) order as the block radix select,
// without barriers.
template <int KP>
__global__ __launch_bounds__(256) void select_probes_wave_kernel(
    const double* __restrict__ cd64, int B, int nlist, int nprobe, int32_t* __restrict__ out_cids,
    float* __restrict__ out_dqcs, int ld, int32_t* __restrict__ out2_cids,
    float* __restrict__ out2_dqcs, int ld2) {
    constexpr int kPer = 16;  // keys per lane per chunk
    __shared__ uint64_t s_ck[kWavesPerBlock][kPer * kWave];
    __shared__ int32_t s_ci[kWavesPerBlock][kPer * kWave];
    const int lane = threadIdx.x & 63;
    const int wid = (int)(threadIdx.x >> 6);
    const int q = blockIdx.x * kWavesPerBlock + wid;
    if (q >= B) return;
    const double* row = cd64 + (size_t)q * nlist;
    uint64_t* ck = s_ck[wid];
    int32_t* ci = s_ci[wid];
    WaveList<KP> L;
    L.init();
    for (int c0 = 0; c0 < nlist; c0 += kPer * kWave) {
        uint64_t k[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = c0 + i * kWave + lane;
            k[i] = c < nlist ? key_of(row[c]) : kKeyInvalid;
        }
        // this lane's smallest and second smallest (key, cid) of the chunk
        uint64_t m1k = kKeyInvalid, m2k = kKeyInvalid;
        int32_t m1i = kIdInvalid, m2i = kIdInvalid;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int32_t id = c0 + i * kWave + lane;
            if (ent_less(k[i], id, m1k, m1i)) {
                m2k = m1k;
                m2i = m1i;
                m1k = k[i];
                m1i = id;
            } else if (ent_less(k[i], id, m2k, m2i)) {
                m2k = k[i];
                m2i = id;
            }
        }
        uint64_t tk = nprobe > kWave ? m2k : m1k;
        int32_t ti = nprobe > kWave ? m2i : m1i;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {  // T0 = max over lanes
            const uint64_t ok = shfl_xor_u64(tk, o);
            const int32_t oi = __shfl_xor(ti, o, kWave);
            if (ent_less(tk, ti, ok, oi)) {
                tk = ok;
                ti = oi;
            }
        }
        uint64_t lk;
        int32_t li;
        L.at(nprobe - 1, lk, li);
        if (ent_less(lk, li, tk, ti)) {
            tk = lk;
            ti = li;
        }
        // compact the entries <= (tk, ti)
        int n = 0;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int32_t id = c0 + i * kWave + lane;
            const bool take = !ent_less(tk, ti, k[i], id) && k[i] != kKeyInvalid;
            const uint64_t m = __ballot(take);
            if (take) {
                const int pos = n + mask_rank(m);
                ck[pos] = k[i];
                ci[pos] = id;
            }
            n += __popcll(m);
        }
        wave_sync();
        for (int b0 = 0; b0 < n; b0 += kWave) {
            const int i = b0 + lane;
            list_offer(L, nprobe, i < n ? ck[i] : kKeyInvalid, i < n ? ci[i] : kIdInvalid);
        }
        wave_sync();
    }
    auto emit = [&](int rank, uint64_t key, int32_t cid) {
        const float dq = (float)sqrt(dist_of(key));
        out_cids[(size_t)q * ld + rank] = cid;
        out_dqcs[(size_t)q * ld + rank] = dq;
        if (out2_cids) out2_cids[(size_t)q * ld2 + rank] = cid;
        if (out2_dqcs) out2_dqcs[(size_t)q * ld2 + rank] = dq;
    };
    if (lane < nprobe) emit(lane, L.k0, L.i0);
    if constexpr (KP == 128) {
        if (kWave + lane < nprobe) emit(kWave + lane, L.k1, L.i1);
    }
}

template __global__ void select_probes_wave_kernel<64>(const double*, int, int, int, int32_t*,
                                                       float*, int, int32_t*, float*, int);
template __global__ void select_probes_wave_kernel<128>(const double*, int, int, int, int32_t*,
                                                        float*, int, int32_t*, float*, int);

// Pair grouping with the histogram aggregated in LDS (used when 2 (nlist + 1) counters fit
// the dynamic LDS): each block counts one chunk of kGroupChunk (query, probe) entries with LDS
// atomics and adds its non-zero bins to the global counts -- one global atomic per (block,
// cluster) instead of one per pair.
__global__ __launch_bounds__(256) void count_pairs_lds_kernel(const int32_t* __restrict__ probe_cids,
                                                              int ld, int B, int nprobe, int p_init,
                                                              int nlist, int32_t* counts) {
    extern __shared__ int32_t s_hist[];
    const int H = 2 * (nlist + 1);
    for (int i = threadIdx.x; i < H; i += blockDim.x) s_hist[i] = 0;
    __syncthreads();
    const int total = B * nprobe;
    const int i0 = blockIdx.x * kGroupChunk, i1 = min(total, i0 + kGroupChunk);
    for (int idx = i0 + (int)threadIdx.x; idx < i1; idx += blockDim.x) {
        const int q = idx / nprobe, p = idx - q * nprobe;
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;  // invalid caller input: never index
        atomicAdd(&s_hist[(p < p_init ? 0 : (nlist + 1)) + cid], 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const int v = s_hist[i];
        if (v) atomicAdd(&counts[i], v);
    }
}

// Same chunks as count_pairs_lds_kernel: the block reserves one range per non-empty bin
// (a global atomicAdd on the cursor) and places its entries with LDS atomics.
__global__ __launch_bounds__(256) void scatter_pairs_lds_kernel(
    const int32_t* __restrict__ probe_cids, const float* __restrict__ probe_dqcs, int ld, int B,
    int nprobe, int p_init, int nlist, int32_t* cursor, int32_t* __restrict__ p1_cids,
    int32_t* __restrict__ p1_qids, float* __restrict__ p1_dqcs, int32_t* __restrict__ p2_cids,
    int32_t* __restrict__ p2_qids, float* __restrict__ p2_dqcs) {
    extern __shared__ int32_t s_hist[];
    const int H = 2 * (nlist + 1);
    for (int i = threadIdx.x; i < H; i += blockDim.x) s_hist[i] = 0;
    __syncthreads();
    const int total = B * nprobe;
    const int i0 = blockIdx.x * kGroupChunk, i1 = min(total, i0 + kGroupChunk);
    for (int idx = i0 + (int)threadIdx.x; idx < i1; idx += blockDim.x) {
        const int q = idx / nprobe, p = idx - q * nprobe;
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;
        atomicAdd(&s_hist[(p < p_init ? 0 : (nlist + 1)) + cid], 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const int v = s_hist[i];
        if (v) s_hist[i] = atomicAdd(&cursor[i], v);
    }
    __syncthreads();
    for (int idx = i0 + (int)threadIdx.x; idx < i1; idx += blockDim.x) {
        const int q = idx / nprobe, p = idx - q * nprobe;
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;
        const bool first = p < p_init;
        const int slot = atomicAdd(&s_hist[(first ? 0 : (nlist + 1)) + cid], 1);
        int32_t* oc = first ? p1_cids : p2_cids;
        int32_t* oq = first ? p1_qids : p2_qids;
        float* od = first ? p1_dqcs : p2_dqcs;
        oc[slot] = cid;
        oq[slot] = q;
        if (od) od[slot] = probe_dqcs ? probe_dqcs[(size_t)q * ld + p] : 0.0f;
    }
}

}  // namespace trident
