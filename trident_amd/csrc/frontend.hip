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

// One counter copied on the stream (a kernel, not a memcpy node, so that a captured graph
// replays it like the kernels around it).
__global__ void copy_u64_kernel(const unsigned long long* src, unsigned long long* dst) {
    if (threadIdx.x == 0) *dst = *src;
}

__global__ void fill_i32_kernel(int32_t* p, int32_t v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// grid (ceil(max(D, D_pad) / 128), ceil(B / (4 kPrepQB))), block (64, 4): each wave takes
// kPrepQB queries (wave-uniform rows, scalar loads) x 128 columns (two per lane), so every
// converted query value feeds two chains and every rotation value kPrepQB.
// xq64[b, d] = (double)xq[b, d]; xrot64[b, j] = sum_d xq[b, d] * R[d, j] + bvec[j] evaluated
// in float64 (fma, dimension order), xrot32 = xrot64 rounded to float32, and qerr[b, j] bounds
// the distance of xrot64 from the exact value: |fl(sum) - sum| <= (D + 1) 2^-53 sum_d |x_d R_dj|
// <= (D + 1) 2^-53 |x| |R_j| (Cauchy-Schwarz; both norms from float64 sums), taken with a
// factor two (and the bias) for the roundings of the norms.
__global__ __launch_bounds__(256) void prep_queries_kernel(
    const float* __restrict__ xq, int B, int D, int D_pad, const float* __restrict__ W, int ldw,
    int nlist, const float* __restrict__ bvec, double* __restrict__ xq64,
    double* __restrict__ xrot64, float* __restrict__ xrot32, double* __restrict__ qerr,
    int do_rot) {
    constexpr int QB = kPrepQB;
    const int lane = threadIdx.x;
    const int j0 = blockIdx.x * 128 + lane, j1 = j0 + 64;
    const int b0 = (blockIdx.y * 4 + threadIdx.y) * QB;
    if (b0 >= B) return;
    const float* qr[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) qr[i] = xq + (size_t)min(b0 + i, B - 1) * D;
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        if (b0 + i >= B) break;
        if (j0 < D) xq64[(size_t)(b0 + i) * D + j0] = (double)qr[i][j0];
        if (j1 < D) xq64[(size_t)(b0 + i) * D + j1] = (double)qr[i][j1];
    }
    if (!do_rot || j0 >= D_pad) return;
    // squared norms of the wave's queries, dims split over the lanes
    double nx[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) {
        double t = 0.0;
        for (int d = lane; d < D; d += kWave) {
            const double v = (double)qr[i][d];
            t = fma(v, v, t);
        }
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) t += __shfl_xor(t, o, kWave);
        nx[i] = t;
    }
    double acc0[QB], acc1[QB], rn0 = 0.0, rn1 = 0.0;
#pragma unroll
    for (int i = 0; i < QB; ++i) acc0[i] = acc1[i] = 0.0;
    const bool h1 = j1 < D_pad;
    const float* wc0 = W + nlist + j0;
    const float* wc1 = W + nlist + (h1 ? j1 : j0);
#pragma unroll 4
    for (int d = 0; d < D; ++d) {
        const double r0 = (double)wc0[(size_t)d * ldw];
        const double r1 = (double)wc1[(size_t)d * ldw];
        rn0 = fma(r0, r0, rn0);
        rn1 = fma(r1, r1, rn1);
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            const double qd = (double)qr[i][d];
            acc0[i] = fma(qd, r0, acc0[i]);
            acc1[i] = fma(qd, r1, acc1[i]);
        }
    }
    auto out = [&](int j, const double (&acc)[QB], double rn) {
        const double bj = (double)bvec[nlist + j];
        const double sr = sqrt(rn);
#pragma unroll
        for (int i = 0; i < QB; ++i) {
            if (b0 + i >= B) break;
            const double xr = acc[i] + bj;
            xrot64[(size_t)(b0 + i) * D_pad + j] = xr;
            xrot32[(size_t)(b0 + i) * D_pad + j] = (float)xr;
            qerr[(size_t)(b0 + i) * D_pad + j] =
                (double)(D + 3) * 0x1p-52 * (sqrt(nx[i]) * sr * (1.0 + 1e-12) + fabs(bj)) +
                0x1p-1000;
        }
    };
    out(j0, acc0, rn0);
    if (h1) out(j1, acc1, rn1);
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

// The cluster-major layout (each cluster's pass-1 pairs, then its pass-2 pairs) from counts
// [2, nlist + 1]: seg_off row 0 = cluster starts, row 1 = pass-2 starts; the cursor rows are the
// same offsets, so the scatter kernels place pass p's pair of cluster c at cursor[p][c]++ in one
// array.  Two launches over ceil(nlist / kBlock) blocks of one cluster per thread (coalesced):
// the first scans each block's clusters and writes the in-block offsets and the block's total,
// the second adds the totals of the blocks before it (at most kBlock blocks).
__global__ __launch_bounds__(256) void scan_pairs_joint_local_kernel(const int32_t* counts,
                                                                     int nlist, int32_t* seg_off,
                                                                     int32_t* blk_tot) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int c = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t n = c < nlist ? (uint32_t)(counts[c] + counts[nlist + 1 + c]) : 0u;
    uint32_t total = 0;
    const uint32_t run = block_exclusive_scan(n, s_wtot, &total);
    if (c < nlist) seg_off[c] = (int32_t)run;
    if (threadIdx.x == 0) blk_tot[blockIdx.x] = (int32_t)total;
}

__global__ __launch_bounds__(256) void scan_pairs_joint_carry_kernel(const int32_t* counts,
                                                                     int nlist,
                                                                     const int32_t* blk_tot,
                                                                     int nblk, int32_t* seg_off,
                                                                     int32_t* cursor) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int tid = threadIdx.x, c = blockIdx.x * kBlock + tid;
    uint32_t total = 0;
    const uint32_t t = tid < nblk ? (uint32_t)blk_tot[tid] : 0u;
    // the exclusive prefix at thread blockIdx.x is this block's carry; broadcast it through LDS
    __shared__ uint32_t s_carry;
    const uint32_t before = block_exclusive_scan(t, s_wtot, &total);
    if (tid == (int)blockIdx.x) s_carry = before;
    __syncthreads();
    if (c < nlist) {
        const uint32_t base = (uint32_t)seg_off[c] + s_carry;
        const uint32_t n1 = (uint32_t)counts[c];
        seg_off[c] = cursor[c] = (int32_t)base;
        seg_off[nlist + 1 + c] = cursor[nlist + 1 + c] = (int32_t)(base + n1);
    }
    if (blockIdx.x == 0 && tid == 0) {
        seg_off[nlist] = cursor[nlist] = (int32_t)total;
        seg_off[2 * nlist + 1] = cursor[2 * nlist + 1] = (int32_t)total;
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

// Large nlist with a rank buffer (B * nprobe entries): the count keeps each pair's arrival
// rank in its bin (the returned counter value), so the scatter places the pair at seg_off[bin]
// + rank with plain loads -- one global atomic per pair instead of two.
__global__ void count_pairs_rank_kernel(const int32_t* __restrict__ probe_cids, int ld, int B,
                                        int nprobe, int p_init, int nlist, int32_t* counts,
                                        int32_t* __restrict__ rank) {
    const int64_t total = (int64_t)B * nprobe;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int q = (int)(idx / nprobe), p = (int)(idx - (int64_t)q * nprobe);
        const int cid = probe_cids[(size_t)q * ld + p];
        if ((unsigned)cid >= (unsigned)nlist) continue;  // invalid caller input: never index
        rank[idx] = atomicAdd(&counts[(p < p_init ? 0 : (nlist + 1)) + cid], 1);
    }
}

__global__ void scatter_pairs_rank_kernel(const int32_t* __restrict__ probe_cids,
                                          const float* __restrict__ probe_dqcs, int ld, int B,
                                          int nprobe, int p_init, int nlist,
                                          const int32_t* __restrict__ seg_off,
                                          const int32_t* __restrict__ rank,
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
        const int slot = seg_off[(first ? 0 : (nlist + 1)) + cid] + rank[idx];
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
    const int i0 = blockIdx.x * kGroupChunk;
    constexpr int kPer = kGroupChunk / 256;  // entries per thread, loads issued together
    int bin[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int idx = i0 + k * 256 + (int)threadIdx.x;
        bin[k] = -1;
        if (idx < total) {
            const int q = idx / nprobe, p = idx - q * nprobe;
            const int cid = probe_cids[(size_t)q * ld + p];
            // invalid caller input: never index
            if ((unsigned)cid < (unsigned)nlist) bin[k] = (p < p_init ? 0 : (nlist + 1)) + cid;
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
        if (bin[k] >= 0) atomicAdd(&s_hist[bin[k]], 1);
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
    const int i0 = blockIdx.x * kGroupChunk;
    constexpr int kPer = kGroupChunk / 256;  // entries per thread, loads issued together
    int bin[kPer], qq[kPer];
    float dq[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int idx = i0 + k * 256 + (int)threadIdx.x;
        bin[k] = -1;
        qq[k] = 0;
        dq[k] = 0.0f;
        if (idx < total) {
            const int q = idx / nprobe, p = idx - q * nprobe;
            const int cid = probe_cids[(size_t)q * ld + p];
            if ((unsigned)cid < (unsigned)nlist) bin[k] = (p < p_init ? 0 : (nlist + 1)) + cid;
            qq[k] = q;
            if (probe_dqcs) dq[k] = probe_dqcs[(size_t)q * ld + p];
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
        if (bin[k] >= 0) atomicAdd(&s_hist[bin[k]], 1);
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const int v = s_hist[i];
        if (v) s_hist[i] = atomicAdd(&cursor[i], v);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        if (bin[k] < 0) continue;
        const bool first = bin[k] <= nlist;
        const int cid = first ? bin[k] : bin[k] - (nlist + 1);
        const int slot = atomicAdd(&s_hist[bin[k]], 1);
        int32_t* oc = first ? p1_cids : p2_cids;
        int32_t* oq = first ? p1_qids : p2_qids;
        float* od = first ? p1_dqcs : p2_dqcs;
        oc[slot] = cid;
        oq[slot] = qq[k];
        if (od) od[slot] = dq[k];
    }
}

// ---------------------------------------------------------------------------------------------
// Band front end (nprobe <= 128): approximate coarse distances on the matrix
// cores with a rigorous error bound, then the canonical float64 distance for the band of
// centroids that can still be among the nprobe nearest, and the exact (d, cid) selection.
//
// For float32 vectors q, c (exact reals) with d = |q - c|^2, nq = |q|^2, nc = |c|^2:
//   s' = the matrix-core float32 dot product of q and c in any summation order, each product
//        and addition with relative error <= 2^-23 (round-to-nearest gives 2^-24; the factor
//        two also covers truncation): |s' - q.c| <= kappa sum |q_d c_d| <= kappa (nq + nc) / 2,
//        kappa = (Dq + 2) 2^-23 (first-order bound of recursive summation over Dq terms);
//   a  = fma(-2, s', fl(nq32 + nc32)) with nq32, nc32 the float64 norms rounded to float32:
//        the three roundings add at most 2^-22 (nq + nc) (1 + 2^-20);
//   d64, the canonical float64 chain, is within 2^-44 (nq + nc) of d.
// So |a - d64| <= E = (kappa + 2^-21) (nq + nc_max) (1 + 2^-10) for every centroid.  If T is
// any value with at least nprobe approximations a <= T, then at least nprobe centroids have
// d64 <= T + E, so the nprobe-th smallest d64 is <= T + E and every centroid of the true
// (d, cid) top-nprobe -- ties included -- has a <= T + 2E.  Those are the band; their exact d64
// decide the selection, exactly as a full float64 pass would.
//
// bfloat16 split form (Dq <= 128, coarse_gemm_bf16_kernel): every float32 value x is split as
// x = h + l + r with h = bf16(x), l = bf16(x - h) (round to nearest even; x - h is exact in
// float32), so |x - h| <= 2^-8 |x|, |l| <= 2^-8 (1 + 2^-8) |x| and |r| <= 2^-16 |x|.  The matrix
// cores sum the exact float32 products h_q h_c, h_q l_c and l_q h_c over the Dp = 32 ceil(Dq / 32)
// (zero-padded) dimensions; the dropped terms l_q l_c + (h_q + l_q) r_c + r_q (h_c + l_c) +
// r_q r_c are at most 3.02 * 2^-16 |q_d c_d| per dimension.  The h h products (<= (1 + 2^-7)
// |q_d c_d|) pass through at most Dp / 2 + 2 additions, the mixed ones (<= 2^-7 (1 + 2^-7)
// |q_d c_d| per pair) through at most Dp + 2, each with relative error <= 2^-23, so
//   kappa = (Dp + 4) 2^-23 (1 + 2^-5) + 3.125 * 2^-16
// bounds |s' - q.c| / sum |q_d c_d| to first order (the margins cover the second-order terms).
// Subnormal bfloat16 operands or float32 products that the matrix cores flush to zero add at
// most 3 Dp 2^-126 (1 + |q|_inf + |c|_inf) <= Dp 2^-100 (1 + nq + nc) in absolute terms.

// Matrix-core tile layout of zero-padded float32 rows (Dq = D rounded up to 16, S = Dq / 4):
// for rows 16 t .. 16 t + 15, float4 number (t S/4 + j) 64 + lane holds, for row 16 t + lane % 16
// and lane group g = lane / 16, dimensions g S + 4 j .. g S + 4 j + 3 -- the A (or B) operands
// of four consecutive v_mfma_f32_16x16x4f32 steps, so one float4 load of a wave is 1 KiB
// contiguous.
__device__ __forceinline__ size_t mfma_tile_offset(int row, int d, int S) {
    const int g = d / S, sd = d - g * S;
    return ((((size_t)(row >> 4) * (S >> 2) + (sd >> 2)) * kWave + (row & 15) + 16 * g) << 2) +
           (sd & 3);
}

// bfloat16 split tile layout (NS 32-dim steps): for rows 16 t .. 16 t + 15, step s and part p
// (0: h, 1: l), the 16 bytes ((t NS + s) 2 + p) 64 + lane hold row 16 t + lane % 16, dimensions
// 32 s + 8 g .. 32 s + 8 g + 7 (g = lane / 16) -- one v_mfma_f32_16x16x32_bf16 operand, read by
// a wave as 1 KiB contiguous.  Returns the offset of (row, d, p) in bfloat16 units.
__device__ __forceinline__ size_t bf16_tile_offset(int row, int d, int NS, int p) {
    const int s = d >> 5, k = d & 31;
    return ((((size_t)(row >> 4) * NS + s) * 2 + p) * kWave + (row & 15) + 16 * (k >> 3)) * 8 +
           (k & 7);
}

// bfloat16 bits of x rounded to nearest even; a finite x that would round to infinity is
// truncated instead (no larger than the float32 products could hold anyway).
__device__ __forceinline__ uint16_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const bool fin = (u & 0x7f800000u) != 0x7f800000u;
    return (uint16_t)(fin && (r & 0x7f80u) == 0x7f80u ? (u >> 16) : r);
}

// x = h + l + r: h = bf16(x), l = bf16(x - h) (x - h is exact in float32)
__device__ __forceinline__ void split_bf16(float x, uint16_t& h, uint16_t& l) {
    h = bf16_rne(x);
    l = bf16_rne(x - __uint_as_float((uint32_t)h << 16));
}

// Queries in the tile layout (qt32) and their squared norms (float64 sum, float32 copy).
__global__ __launch_bounds__(256) void pad_queries_kernel(const float* __restrict__ xq, int B,
                                                          int D, int Dq,
                                                          float* __restrict__ qt32,
                                                          float* __restrict__ qn32, int NS,
                                                          uint16_t* __restrict__ qtb) {
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    if (q >= B) return;
    const int S = Dq >> 2;
    double acc = 0.0;
    for (int d = lane; d < Dq; d += kWave) {
        const float v = d < D ? xq[(size_t)q * D + d] : 0.0f;
        if (qt32) qt32[mfma_tile_offset(q, d, S)] = v;
        acc = fma((double)v, (double)v, acc);
    }
    if (qtb) {  // the bfloat16 split layout (NS 32-dim steps, zero past D)
        for (int d = lane; d < 32 * NS; d += kWave) {
            uint16_t h, l;
            split_bf16(d < D ? xq[(size_t)q * D + d] : 0.0f, h, l);
            qtb[bf16_tile_offset(q, d, NS, 0)] = h;
            qtb[bf16_tile_offset(q, d, NS, 1)] = l;
        }
    }
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) acc += __shfl_xor(acc, o, kWave);
    if (lane == 0) qn32[q] = (float)acc;
}

// Centroids (c_d = -0.5f W[d, c], the same float32 values the float64 chains use) as
// centroid-major zero-padded rows cm32 [nlist, Dq] and in the tile layout (cmt32), their
// squared norms cn32 (float64 partial sums rounded to float32: only the error bound and the
// approximations use them) and the largest squared norm (float64 bit pattern, atomicMax into a
// cell the caller zeroes).  grid ceil(nlist / 64), block 256: 64 centroids per block,
// transposed through LDS in 64-dim tiles (W rows read and cm32 rows written coalesced).
__global__ __launch_bounds__(256) void pad_centroids_kernel(const float* __restrict__ W, int ldw,
                                                            int nlist, int D, int Dq,
                                                            float* __restrict__ cm32,
                                                            float* __restrict__ cmt32,
                                                            float* __restrict__ cn32,
                                                            unsigned long long* __restrict__ cmax2) {
    __shared__ float s_t[64][65];
    __shared__ double s_n[4][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int c0 = blockIdx.x * 64;
    const int S = Dq >> 2;
    double nrm = 0.0;  // centroid c0 + tx over dims ty, ty + 4, ...
    for (int d0 = 0; d0 < Dq; d0 += 64) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {  // s_t[d][c] = centroid c0 + c, dim d0 + d
            const int r = ty + 4 * k, d = d0 + r, c = c0 + tx;
            const float v = (d < D && c < nlist) ? -0.5f * W[(size_t)d * ldw + c] : 0.0f;
            s_t[r][tx] = v;
            nrm = fma((double)v, (double)v, nrm);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; ++k) {  // centroid c0 + r, dim d0 + tx
            const int r = ty + 4 * k, c = c0 + r, d = d0 + tx;
            if (c < nlist && d < Dq) {
                const float v = s_t[tx][r];
                cm32[(size_t)c * Dq + d] = v;
                cmt32[mfma_tile_offset(c, d, S)] = v;
            }
        }
        __syncthreads();
    }
    s_n[ty][tx] = nrm;
    __syncthreads();
    if (ty == 0) {
        double n = 0.0;
        if (c0 + tx < nlist) {
            n = (s_n[0][tx] + s_n[1][tx]) + (s_n[2][tx] + s_n[3][tx]);
            cn32[c0 + tx] = (float)n;
        }
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) n = fmax(n, __shfl_xor(n, o, kWave));
        // one atomic per block: same-address atomics serialise in L2
        if (tx == 0) atomicMax(cmax2, (unsigned long long)__double_as_longlong(n));
    }
}

// One-dimensional grid of 8 * ceil(B / 64) * ceil(ncg / 8) blocks (ncg = ceil(nlist / (16
// kGemmTiles)) centroid groups), block 256.  Blocks are dealt to the XCDs round-robin, so block
// b runs on XCD b % 8: XCD x takes centroid groups [x cpx, (x + 1) cpx) (cpx = ceil(ncg / 8)) for
// every query block, and its share of the centroid tiles stays in its L2.  Used for Dq > 128
// (coarse_gemm_bf16_kernel takes Dq <= 128).  Each wave 16 queries (one query tile), all four
// waves the same kGemmTiles centroid tiles in the same order.  v_mfma_f32_16x16x4f32 with query
// rows as A (16 x 4) and centroids as B (4 x 16), operands straight from the tile layouts: a
// chunk of 32 k-steps is 8 + 8 coalesced float4 loads, issued whole before its 32 MFMAs; steps
// past S are zero (clamped loads, no branch among the MFMAs).
// a32[q, c] = fma(-2, dot, nq32 + nc32).
__global__ __launch_bounds__(256) void coarse_gemm_kernel(const float* __restrict__ qt32,
                                                          const float* __restrict__ qn32, int B,
                                                          const float* __restrict__ cmt32,
                                                          const float* __restrict__ cn32,
                                                          int nlist, int Dq,
                                                          float* __restrict__ a32) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m = lane & 15, g = lane >> 4;
    const int ncg = (nlist + 16 * kGemmTiles - 1) / (16 * kGemmTiles), cpx = (ncg + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7), local = (int)(blockIdx.x >> 3);
    const int bx = local / cpx, by = xcd * cpx + (local - (local / cpx) * cpx);
    if (by >= ncg || bx * 64 >= B) return;  // the whole block
    const int qb0 = bx * 64 + wid * 16;
    const bool wave_live = qb0 < B;
    const int qtile = wave_live ? qb0 / 16 : 0;
    const int qb = wave_live ? qb0 : 0;
    const int F = Dq >> 4;  // float4 per lane and row tile (= S / 4)
    const float4* qt = reinterpret_cast<const float4*>(qt32) + (size_t)qtile * F * kWave + lane;
    const bool qv = wave_live && qb + m < B;
    auto store = [&](int n0, const f4 (&acc4)[4]) {
        // matrix-core results: wait states before the first VALU read, fenced
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7");
        __builtin_amdgcn_sched_barrier(0);
        const f4 acc = (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
        const int c = n0 + m;
        if (c < nlist) {
            const float ncv = cn32[c];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = qb + 4 * g + i;
                if (q < B) a32[(size_t)q * nlist + c] = fmaf(-2.0f, acc[i], qn32[q] + ncv);
            }
        }
    };
    if (!wave_live) return;
#pragma unroll 1
    for (int t = 0; t < kGemmTiles; ++t) {
        const int n0 = by * 16 * kGemmTiles + t * 16;
        if (n0 >= nlist) break;
        const bool cv = n0 + m < nlist;
        const float4* ct = reinterpret_cast<const float4*>(cmt32) + (size_t)(n0 >> 4) * F * kWave +
                           lane;
        // four independent accumulator chains (k-step 4 j + u -> chain u), summed at the end:
        // the error bound holds for any summation order
        f4 acc4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc4[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
        for (int f0 = 0; f0 < F; f0 += 8) {
            float4 av[8], bv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool in = f0 + j < F;
                const size_t o = (size_t)(in ? f0 + j : 0) * kWave;
                av[j] = qt[o];
                bv[j] = ct[o];
                if (!in || !qv) av[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (!cv) bv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].x, bv[j].x, acc4[0], 0, 0, 0);
                acc4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].y, bv[j].y, acc4[1], 0, 0, 0);
                acc4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].z, bv[j].z, acc4[2], 0, 0, 0);
                acc4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j].w, bv[j].w, acc4[3], 0, 0, 0);
            }
        }
        store(n0, acc4);
    }
}


// Centroid rows cm32 [nlist, Dq] -> the bfloat16 split tile layout (NS steps), rows up to the
// next multiple of 16 and dimensions past Dq zero.  One thread per (row, dimension pair).
__global__ __launch_bounds__(256) void centroid_bf16_kernel(const float* __restrict__ cm32,
                                                            int nlist, int Dq, int NS,
                                                            uint32_t* __restrict__ cmtb) {
    const int npair = 16 * NS;  // dimension pairs per row
    const int64_t n = (int64_t)((nlist + 15) & ~15) * npair;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int row = (int)(i / npair), d = 2 * (int)(i - (int64_t)row * npair);
        const float* src = cm32 + (size_t)row * Dq;
        uint16_t h0, l0, h1, l1;
        split_bf16(row < nlist && d < Dq ? src[d] : 0.0f, h0, l0);
        split_bf16(row < nlist && d + 1 < Dq ? src[d + 1] : 0.0f, h1, l1);
        // d even: (d, d + 1) share one 32-bit word of each part
        cmtb[bf16_tile_offset(row, d, NS, 0) >> 1] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        cmtb[bf16_tile_offset(row, d, NS, 1) >> 1] = (uint32_t)l0 | ((uint32_t)l1 << 16);
    }
}

// Dq <= 128: the coarse pass on the bfloat16 matrix cores, with a block's query tiles kept for a
// run of centroid stages.  One-dimensional grid of 8 * ceil(B / 64) * nrun blocks: block b runs
// on XCD x = b % 8 and takes query block bx and run r of XCD x's share of the stages
// (kStageTiles 16-centroid tiles each; XCD x owns stages [x spx, (x + 1) spx), split into nrun
// runs of run_stages), so its centroid tiles stay in its L2.  The four waves' split query
// operands (NS 32-dim steps, 2 NS 16-byte operands per lane and row tile) stay in registers for
// the whole run; each stage's tiles are fetched into registers while the waves compute the
// previous stage from LDS, then written to the other LDS buffer.  Per tile four independent
// accumulator chains: h h products of even and odd steps, and h l, l h products;
// a = fma(-2, (H0 + H1) + (L0 + L1), nq32 + nc32), in rows of lda = nlist rounded up to 4 floats
// (the padding is never read); with tmin, also each query's 16-centroid tile minima.
template <int NS>
__global__ __launch_bounds__(256) void coarse_gemm_bf16_kernel(const uint32_t* __restrict__ qtb,
                                                               const float* __restrict__ qn32,
                                                               int B,
                                                               const uint32_t* __restrict__ cmtb,
                                                               const float* __restrict__ cn32,
                                                               int nlist, int run_stages,
                                                               float* __restrict__ a32,
                                                               float* __restrict__ tmin) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    constexpr int U = 2 * NS;                                            // u4 per lane and tile
    constexpr int PT = (kStageTiles * U * kWave + kBlock - 1) / kBlock;  // u4 per thread, stage
    static_assert(NS >= 1 && NS <= 4, "Dq <= 128");
    static_assert(PT >= 1 && PT <= 4, "at most four u4 per thread and stage");
    __shared__ u4 s_b[2][PT * kBlock];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m = lane & 15, g = lane >> 4;
    const int ntl_all = (nlist + 15) / 16;
    const int lda = band_lda(nlist);
    const int nst = (ntl_all + kStageTiles - 1) / kStageTiles, spx = (nst + 7) >> 3;
    const int nrun = (spx + run_stages - 1) / run_stages;
    const int xcd = (int)(blockIdx.x & 7), local = (int)(blockIdx.x >> 3);
    const int bx = local / nrun, run = local - bx * nrun;
    const int s_beg = xcd * spx + run * run_stages;
    const int s_end = min(min(s_beg + run_stages, (xcd + 1) * spx), nst);
    if (s_beg >= s_end || bx * 64 >= B) return;  // the whole block
    const int qb0 = bx * 64 + wid * 16;
    const bool wave_live = qb0 < B;  // waves past the last query still load and wait
    const int qtile = wave_live ? qb0 / 16 : 0;
    const int qb = wave_live ? qb0 : 0;
    u4 av[U];  // rows past B are never stored
    {
        const u4* qt = reinterpret_cast<const u4*>(qtb) + (size_t)qtile * U * kWave + lane;
#pragma unroll
        for (int j = 0; j < U; ++j) av[j] = qt[(size_t)j * kWave];
    }
    const u4* cb = reinterpret_cast<const u4*>(cmtb);
    // thread i moves u4s i, i + 256, ... of a stage's contiguous run (slots past the stage's
    // tiles are never read: they load element 0 again)
    u4 r[PT];
    auto fetch = [&](int st) __attribute__((always_inline)) {
        const int t0 = st * kStageTiles, n = min(kStageTiles, ntl_all - t0) * U * kWave;
        const u4* p = cb + (size_t)t0 * U * kWave;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int i = (int)threadIdx.x + k * kBlock;
            r[k] = p[i < n ? i : 0];
        }
    };
    auto put = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < PT; ++k) s_b[b][threadIdx.x + k * kBlock] = r[k];
    };
    // tile minima (tmin, when not null: [B, ceil(nlist / 16)]) of the current 16-tile chunk:
    // lane (m, g) holds tiles 16 ch + 4 g + [0, 4) of query qb + m, written as one 16-byte store
    // per lane when the chunk moves on (tiles outside this block's run are left to the blocks
    // that run them)
    const int tile_lo = s_beg * kStageTiles, tile_hi = min(s_end * kStageTiles, ntl_all);
    float mt0 = INFINITY, mt1 = INFINITY, mt2 = INFINITY, mt3 = INFINITY;
    int chunk = -1;
    auto flush_mt = [&]() __attribute__((always_inline)) {
        const int q = qb + m, tb = 16 * chunk + 4 * g;
        if (!tmin || chunk < 0 || q >= B) return;
        float* dst = tmin + (size_t)q * ntl_all + tb;
        if ((ntl_all & 3) == 0 && tb >= tile_lo && tb + 4 <= tile_hi) {
            *reinterpret_cast<float4*>(dst) = make_float4(mt0, mt1, mt2, mt3);
        } else {
            const float mv[4] = {mt0, mt1, mt2, mt3};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (tb + i >= tile_lo && tb + i < tile_hi) dst[i] = mv[i];
        }
    };
    fetch(s_beg);
    put(0);
    __syncthreads();
    for (int st = s_beg; st < s_end; ++st) {
        const int buf = (st - s_beg) & 1;
        if (st + 1 < s_end) fetch(st + 1);
        if (wave_live) {
            const int t0 = st * kStageTiles, ntl = min(kStageTiles, ntl_all - t0);
#pragma unroll 1
            for (int t = 0; t < ntl; ++t) {
                u4 bv[U];
#pragma unroll
                for (int j = 0; j < U; ++j) bv[j] = s_b[buf][(t * U + j) * kWave + lane];
                // centroids are the A operand, queries the B operand
                f4 h0 = {0.0f, 0.0f, 0.0f, 0.0f}, h1 = h0, l0 = h0, l1 = h0;
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const bf8 cH = __builtin_bit_cast(bf8, bv[2 * s]),
                              cL = __builtin_bit_cast(bf8, bv[2 * s + 1]);
                    const bf8 qH = __builtin_bit_cast(bf8, av[2 * s]),
                              qL = __builtin_bit_cast(bf8, av[2 * s + 1]);
                    if (s & 1) h1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cH, qH, h1, 0, 0, 0);
                    else h0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cH, qH, h0, 0, 0, 0);
                    l0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cH, qL, l0, 0, 0, 0);
                    l1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cL, qH, l1, 0, 0, 0);
                }
                const f4 acc = (h0 + h1) + (l0 + l1);
                // lane (m, g) holds centroids 16 (t0 + t) + 4 g .. + 3 of query qb + m
                const int q = qb + m, c0 = 16 * (t0 + t) + 4 * g;
                const float nq = q < B ? qn32[q] : 0.0f;
                float4 nc;
                if ((nlist & 3) == 0 && c0 + 4 <= nlist) {
                    nc = *reinterpret_cast<const float4*>(cn32 + c0);
                } else {
                    nc.x = c0 < nlist ? cn32[c0] : 0.0f;
                    nc.y = c0 + 1 < nlist ? cn32[c0 + 1] : 0.0f;
                    nc.z = c0 + 2 < nlist ? cn32[c0 + 2] : 0.0f;
                    nc.w = c0 + 3 < nlist ? cn32[c0 + 3] : 0.0f;
                }
                const float ncv[4] = {nc.x, nc.y, nc.z, nc.w};
                float o[4], mn = INFINITY;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[i] = fmaf(-2.0f, acc[i], nq + ncv[i]);
                    if (c0 + i < nlist) mn = fminf(mn, o[i]);
                }
                // rows of lda = nlist rounded up to 4 floats: one aligned 16-byte store
                // (c0 < nlist: c0 and lda are multiples of 4, so c0 + 4 <= lda)
                if (q < B && c0 < nlist)
                    *reinterpret_cast<float4*>(a32 + (size_t)q * lda + c0) = make_float4(o[0], o[1], o[2], o[3]);
                if (tmin) {
                    // the tile's minimum for query q (lanes m, m + 16, m + 32, m + 48), kept by lane
                    // group (tile / 4) % 4 in slot tile % 4
                    mn = fminf(mn, __shfl_xor(mn, 16, kWave));
                    mn = fminf(mn, __shfl_xor(mn, 32, kWave));
                    const int tt = t0 + t;
                    if ((tt >> 4) != chunk) {
                        flush_mt();
                        chunk = tt >> 4;
                        mt0 = mt1 = mt2 = mt3 = INFINITY;
                    }
                    if (g == ((tt >> 2) & 3)) {
                        const int sl = tt & 3;
                        mt0 = sl == 0 ? mn : mt0;
                        mt1 = sl == 1 ? mn : mt1;
                        mt2 = sl == 2 ? mn : mt2;
                        mt3 = sl == 3 ? mn : mt3;
                    }
                }
            }
        }
        if (st + 1 < s_end) put(buf ^ 1);
        __syncthreads();
    }
    if (wave_live) flush_mt();
}

template __global__ void coarse_gemm_bf16_kernel<1>(const uint32_t*, const float*, int,
                                                    const uint32_t*, const float*, int, int, float*, float*);
template __global__ void coarse_gemm_bf16_kernel<2>(const uint32_t*, const float*, int,
                                                    const uint32_t*, const float*, int, int, float*, float*);
template __global__ void coarse_gemm_bf16_kernel<3>(const uint32_t*, const float*, int,
                                                    const uint32_t*, const float*, int, int, float*, float*);
template __global__ void coarse_gemm_bf16_kernel<4>(const uint32_t*, const float*, int,
                                                    const uint32_t*, const float*, int, int, float*, float*);

// One wave per query: V approximations per lane (nlist <= 64 V), or, STREAM (any nlist), the
// row streamed through a running filter.  T is any value with count(a <= T) >= nprobe over the
// row: then every centroid among the nprobe nearest (by the exact distance) lies in the band
// a <= T + 2E, and every centroid of the band gets its canonical float64 distance (t = q_d -
// c_d, acc = fma(t, t, acc) in dimension order -- the oracle's chain).  Without STREAM, T comes
// from a bisection on the register values.  STREAM: the wave appends each approximation a <=
// cut = T + 2E of the row to an LDS list (ballot + mbcnt); T starts at +inf and, whenever the
// list fills, becomes the result of a bisection over the list (count(a <= T) >= nprobe over
// the list, so over the row), and entries above the new cut are dropped.  Values dropped or
// never listed lie above every later cut, so the list holds every approximation <= the final
// cut and counts over it equal the row's below that cut: the final bisection runs on the list.
// A list that cannot shrink below half its capacity (a band of more than ~512 centroids) ends
// the filter: the band is then taken from the row again with cut = T + 2E for the T reached.
// A band of <= 128 (the usual case: a few more than nprobe) is ranked by counting, each entry
// against all others in (d, cid) order; a wider one streams through the (d, cid) register list
// 64 centroids at a time.  Outputs as select_probes_wave_kernel.  Row q of a32 starts at
// q lda; STREAM with tmin first filters the row's tile minima (below).
template <int KP, int V, bool STREAM>
__global__ __launch_bounds__(256) void select_band_kernel(
    const float* __restrict__ a32, const double* __restrict__ xq64, const float* __restrict__ cm32,
    const unsigned long long* __restrict__ cmax_dev, double cmax_host, int B, int nlist, int D,
    int Dq, double kappa, double kabs, const float* __restrict__ tmin, int lda, int nprobe,
    int32_t* __restrict__ out_cids, float* __restrict__ out_dqcs, int ld,
    int32_t* __restrict__ out2_cids, float* __restrict__ out2_dqcs, int ld2) {
    // the band's centroids (up to 8 per lane); STREAM: the filter's list (up to 16 per lane),
    // its centroids in s_band and its approximations in s_lval
    constexpr int kBandMax = 8 * kWave;
    constexpr int kListPer = 16, kListCap = kListPer * kWave;
    __shared__ int32_t s_band[kWavesPerBlock][STREAM ? kListCap : kBandMax];
    __shared__ float s_lval[kWavesPerBlock][STREAM ? kListCap : 1];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = blockIdx.x * kWavesPerBlock + wid;
    if (q >= B) return;
    const double* qrow = xq64 + (size_t)q * D;
    const float* arow = a32 + (size_t)q * lda;
    int32_t* band = s_band[wid];
    // the error bound E (float64, then rounded up to float32)
    double nq = 0.0;
    for (int d = lane; d < D; d += kWave) nq = fma(qrow[d], qrow[d], nq);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) nq += __shfl_xor(nq, o, kWave);
    // kappa: the dot product's relative bound of the pass that wrote a32, kabs its absolute
    // term per unit of 1 + nq + nc (float32 operands: (Dq + 2) 2^-23 and 0; bfloat16 split)
    const double cmax2 = cmax_dev ? __longlong_as_double((long long)*cmax_dev) : cmax_host;
    const double E = (kappa + 0x1p-21) * (nq + cmax2) * (1.0 + 0x1p-10) +
                     kabs * (1.0 + nq + cmax2) + 1e-30;
    const float Ef = __double2float_ru(E);
    // E carries a 2^-10 relative margin, which covers the float64 rounding of this sum
    auto cut_of = [&](float t) { return __double2float_ru((double)t + 2.0 * E); };
    // bisection over values held N per lane: count(a <= hi) >= nprobe throughout (hi starts at
    // hi0, or at the largest value when hi0 is +inf); stops once the count is at most nprobe
    // + slack or the interval is no wider than Ef.  Counts come from ballots.
    auto bisect = [&](const float* w, auto n_c, float hi0, int slack) __attribute__((always_inline)) {
        constexpr int N = decltype(n_c)::value;
        float lmin = INFINITY, lmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            lmin = fminf(lmin, w[i]);
            if (w[i] < INFINITY) lmax = fmaxf(lmax, w[i]);
        }
        float lo = lmin, hi = lmax;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            lo = fminf(lo, __shfl_xor(lo, o, kWave));
            hi = fmaxf(hi, __shfl_xor(hi, o, kWave));
        }
        hi = fminf(hi, hi0);
        for (int it = 0; it < 40 && hi - lo > Ef; ++it) {
            const float mid = lo + 0.5f * (hi - lo);
            if (!(mid > lo && mid < hi)) break;
            int n = 0;
#pragma unroll
            for (int i = 0; i < N; ++i) n += __popcll(__ballot(w[i] <= mid));
            if (n >= nprobe) {
                hi = mid;
                if (n <= nprobe + slack) break;
            } else {
                lo = mid;
            }
        }
        return hi;
    };
    float v[STREAM ? 1 : V];
    auto count_le = [&](float x) {
        int n = 0;
#pragma unroll
        for (int i = 0; i < (STREAM ? 1 : V); ++i) n += __popcll(__ballot(v[i] <= x));
        return n;
    };
    float thr;
    int mband = nlist + 1, nb_stream = 0;
    bool from_regs = false;
    if constexpr (STREAM) {
        float* lval = s_lval[wid];
        float T = INFINITY, cut = INFINITY;
        int n = 0;
        bool open = true;
        // the list's entries lane + 64 i into registers (+inf past n)
        auto load_list = [&](float (&w)[kListPer]) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < kListPer; ++i) {
                const int e = i * kWave + lane;
                w[i] = e < n ? lval[e] : INFINITY;
            }
        };
        // keeps the entries <= c, in list order
        auto compact = [&](const float (&w)[kListPer], float c) __attribute__((always_inline)) {
            int32_t id[kListPer];
#pragma unroll
            for (int i = 0; i < kListPer; ++i) id[i] = band[min(i * kWave + lane, kListCap - 1)];
            wave_sync();
            int m = 0;
#pragma unroll
            for (int i = 0; i < kListPer; ++i) {
                // slots past n are never kept (c may be +inf when E overflows)
                const bool keep = i * kWave + lane < n && w[i] <= c;
                const uint64_t mk = __ballot(keep);
                if (keep) {
                    lval[m + mask_rank(mk)] = w[i];
                    band[m + mask_rank(mk)] = id[i];
                }
                m += __popcll(mk);
            }
            wave_sync();
            n = m;
        };
        // before a round that can add `room` entries: tighten T over the list (bisection, then
        // the entries above the new cut dropped); false when the list cannot shrink below
        // kListCap - room (the filter closes)
        auto tighten = [&](int room) __attribute__((always_inline)) {
            if (n <= kListCap - room) return true;
            float w[kListPer];
            wave_sync();
            load_list(w);
            T = bisect(w, std::integral_constant<int, kListPer>{}, T, 32);
            cut = cut_of(T);
            compact(w, cut);
            if (n <= kListCap - room) return true;
            open = false;
            return false;
        };
        // streams src[0, len) through the list (entry ids: the indices): eight of the lane's
        // values per round, all loaded before the first is filtered, and the next round's loaded
        // before this round is filtered
        auto stream = [&](const float* src, int len) __attribute__((always_inline)) {
            auto load8 = [&](float (&x)[8], int c0) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int c = c0 + u * kWave + lane;
                    x[u] = c < len ? src[c] : INFINITY;
                }
            };
            float xn[8];
            load8(xn, 0);
            for (int c0 = 0; c0 < len; c0 += 8 * kWave) {
                if (!tighten(8 * kWave)) break;
                float xs[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) xs[u] = xn[u];
                if (c0 + 8 * kWave < len) load8(xn, c0 + 8 * kWave);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const bool take = c0 + u * kWave + lane < len && xs[u] <= cut;
                    const uint64_t mk = __ballot(take);
                    if (mk == 0ull) continue;
                    if (take) {
                        const int at = n + mask_rank(mk);
                        lval[at] = xs[u];
                        band[at] = c0 + u * kWave + lane;
                    }
                    n += __popcll(mk);
                }
            }
        };
        // With the coarse pass's 16-centroid tile minima (tmin), those first: T with
        // count(tile minimum <= T) >= nprobe over them has count(a <= T) >= nprobe over the row
        // (one centroid per tile at least) and sits near the row's nprobe-th value.  Every
        // approximation a <= cut lies in a tile whose minimum is <= cut, and the filter over the
        // minima ends with all of those tiles listed: only their 16 values each are read (one
        // listed tile per lane at a time).  More than 512 such tiles (a wide band) fall back to
        // streaming the whole row from the T reached, a closed tile filter from T = +inf.
        const int ntl = (nlist + 15) >> 4;
        bool whole_row = true;
        if (tmin && ntl >= nprobe) {
            stream(tmin + (size_t)q * ntl, ntl);
            if (open) {
                float w[kListPer];
                wave_sync();
                load_list(w);
                T = bisect(w, std::integral_constant<int, kListPer>{}, T, 2);
                cut = cut_of(T);
                compact(w, cut);
                if (n <= 8 * kWave) {
                    whole_row = false;
                    int tl[8];  // listed tile lane + 64 k (-1 past the list)
#pragma unroll
                    for (int k = 0; k < 8; ++k) tl[k] = k * kWave + lane < n ? band[k * kWave + lane] : -1;
                    const int n1 = n;
                    n = 0;
                    wave_sync();
#pragma unroll 1
                    for (int k = 0; k < 8; ++k) {
                        if (k * kWave >= n1) break;
                        int tk = tl[0];  // tl[k] by a select chain (no indexed register array)
#pragma unroll
                        for (int j = 1; j < 8; ++j) tk = k == j ? tl[j] : tk;
                        const int c0 = 16 * tk;
                        float xv[16];
#pragma unroll
                        for (int i = 0; i < 16; ++i) xv[i] = tk >= 0 && c0 + i < nlist ? arow[c0 + i] : INFINITY;
                        auto filter8 = [&](auto off_c) __attribute__((always_inline)) {
                            constexpr int O = decltype(off_c)::value;
#pragma unroll
                            for (int i = O; i < O + 8; ++i) {
                                const bool take = xv[i] <= cut;
                                const uint64_t mk = __ballot(take);
                                if (take) {
                                    const int at = n + mask_rank(mk);
                                    lval[at] = xv[i];
                                    band[at] = c0 + i;
                                }
                                n += __popcll(mk);
                            }
                        };
                        if (!tighten(8 * kWave)) break;
                        filter8(std::integral_constant<int, 0>{});
                        if (!tighten(8 * kWave)) break;
                        filter8(std::integral_constant<int, 8>{});
                    }
                } else {
                    n = 0;
                    wave_sync();
                }
            } else {
                T = cut = INFINITY;
                open = true;
                n = 0;
                wave_sync();
            }
        }
        if (whole_row) stream(arow, nlist);
        if (open) {
            float w[kListPer];
            wave_sync();
            load_list(w);
            const float hi = bisect(w, std::integral_constant<int, kListPer>{}, T, 2);
            thr = cut_of(hi);
            compact(w, thr);  // the band, in LDS
            mband = nb_stream = n;
            from_regs = true;
        } else {
            thr = cut;  // T is valid for the row: the band is taken from the row again
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int c = i * kWave + lane;
            v[i] = c < nlist ? arow[c] : INFINITY;
        }
        // hi starts at the largest lane minimum when every lane holds a value and nprobe <= 64
        // (then >= 64 values lie at or below it), else at the largest value
        float t0 = INFINITY;
        {
            float lmin = INFINITY;
#pragma unroll
            for (int i = 0; i < V; ++i) lmin = fminf(lmin, v[i]);
            t0 = lmin;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) t0 = fmaxf(t0, __shfl_xor(t0, o, kWave));
        }
        const float hi = bisect(v, std::integral_constant<int, V>{},
                                nprobe <= kWave && t0 < INFINITY ? t0 : INFINITY, 2);
        thr = cut_of(hi);
    }
    auto emit = [&](int rank, uint64_t key, int32_t cid) {
        const float dq = (float)sqrt(dist_of(key));
        out_cids[(size_t)q * ld + rank] = cid;
        out_dqcs[(size_t)q * ld + rank] = dq;
        if (out2_cids) out2_cids[(size_t)q * ld2 + rank] = cid;
        if (out2_dqcs) out2_dqcs[(size_t)q * ld2 + rank] = dq;
    };
    // canonical float64 distance of centroid c: dimension order, t = q_d - c_d, fma(t, t, acc).
    // The row arrives in chunks of 64 (then 16) dims whose loads are all issued before their
    // first use: one memory round trip per chunk instead of one per 4 dims.
    auto exact = [&](int c) {
        const float* crow = cm32 + (size_t)c * Dq;
        double acc = 0.0;
        int d = 0;
        auto chunk = [&](auto nq4) {
            constexpr int N4 = decltype(nq4)::value;
            float4 cv[N4];
#pragma unroll
            for (int k = 0; k < N4; ++k) cv[k] = *reinterpret_cast<const float4*>(crow + d + 4 * k);
#pragma unroll
            for (int k = 0; k < N4; ++k) {
                double t = qrow[d + 4 * k] - (double)cv[k].x;
                acc = fma(t, t, acc);
                t = qrow[d + 4 * k + 1] - (double)cv[k].y;
                acc = fma(t, t, acc);
                t = qrow[d + 4 * k + 2] - (double)cv[k].z;
                acc = fma(t, t, acc);
                t = qrow[d + 4 * k + 3] - (double)cv[k].w;
                acc = fma(t, t, acc);
            }
            d += 4 * N4;
        };
        while (d + 64 <= D) chunk(std::integral_constant<int, 16>{});
        while (d + 16 <= D) chunk(std::integral_constant<int, 4>{});
        for (; d + 4 <= D; d += 4) {
            const float4 cv = *reinterpret_cast<const float4*>(crow + d);
            double t = qrow[d] - (double)cv.x;
            acc = fma(t, t, acc);
            t = qrow[d + 1] - (double)cv.y;
            acc = fma(t, t, acc);
            t = qrow[d + 2] - (double)cv.z;
            acc = fma(t, t, acc);
            t = qrow[d + 3] - (double)cv.w;
            acc = fma(t, t, acc);
        }
        for (; d < D; ++d) {
            const double t = qrow[d] - (double)crow[d];
            acc = fma(t, t, acc);
        }
        return acc;
    };
    // The band is in LDS (from_regs) when the registers held all of it and it fit kBandMax,
    // or, STREAM, when the filter's list held it.  Otherwise, STREAM, it is compacted from the
    // row in one more pass (eight values per lane loaded per round), counting past the 128
    // slots without writing.
    if constexpr (STREAM) {
        if (!from_regs) {
            for (int c0 = 0; c0 < nlist; c0 += 8 * kWave) {
                float xs[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int c = c0 + u * kWave + lane;
                    xs[u] = c < nlist ? arow[c] : INFINITY;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const bool take = xs[u] <= thr;  // +inf past nlist never passes
                    const uint64_t mk = __ballot(take);
                    const int at = nb_stream + mask_rank(mk);
                    if (take && at < 2 * kWave) band[at] = c0 + u * kWave + lane;
                    nb_stream += __popcll(mk);
                }
            }
            mband = nb_stream;
        }
    } else if (thr < INFINITY) {
        // (not past V = 32: the unrolled compaction would cost a wave per SIMD)
        if (V <= 32 && count_le(thr) <= kBandMax) {
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const bool take = v[i] <= thr;
                const uint64_t mk = __ballot(take);
                if (take) band[nb_stream + mask_rank(mk)] = i * kWave + lane;
                nb_stream += __popcll(mk);
            }
            mband = nb_stream;
            from_regs = true;
        } else {
            mband = count_le(thr);
        }
    }
    if (mband <= 2 * kWave) {
        // the common case: the band fits two entries per lane.  Compact it, compute the exact
        // distances, and rank every entry by counting the entries before it in (d, cid) order.
        int nb = 0;
        if constexpr (STREAM) {
            nb = nb_stream;  // compacted above
        } else if (from_regs) {
            nb = nb_stream;
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const bool take = v[i] <= thr;  // thr is finite: centroids past nlist hold +inf
                const uint64_t mk = __ballot(take);
                if (take) band[nb + mask_rank(mk)] = i * kWave + lane;
                nb += __popcll(mk);
            }
        }
        wave_sync();
        const bool h0 = lane < nb, h1 = kWave + lane < nb;
        const int c0 = band[h0 ? lane : 0], c1 = band[h1 ? kWave + lane : 0];
        const uint64_t k0 = h0 ? key_of(exact(c0)) : kKeyInvalid;
        const uint64_t k1 = h1 ? key_of(exact(c1)) : kKeyInvalid;
        int r0 = 0, r1 = 0;
        if (nb <= kWave) {
            for (int jl = 0; jl < nb; ++jl) {
                const uint64_t kj = readlane_u64(k0, jl);
                r0 += ent_less(kj, __builtin_amdgcn_readlane(c0, jl), k0, c0) ? 1 : 0;
            }
        } else {
            for (int jl = 0; jl < kWave; ++jl) {
                const uint64_t kj = readlane_u64(k0, jl);
                const int32_t cj = __builtin_amdgcn_readlane(c0, jl);
                r0 += ent_less(kj, cj, k0, c0) ? 1 : 0;
                r1 += ent_less(kj, cj, k1, c1) ? 1 : 0;
            }
        }
        for (int jl = 0; jl < nb - kWave; ++jl) {
            const uint64_t kj = readlane_u64(k1, jl);
            const int32_t cj = __builtin_amdgcn_readlane(c1, jl);
            r0 += ent_less(kj, cj, k0, c0) ? 1 : 0;
            r1 += ent_less(kj, cj, k1, c1) ? 1 : 0;
        }
        if (h0 && r0 < nprobe) emit(r0, k0, c0);
        if (h1 && r1 < nprobe) emit(r1, k1, c1);
        return;
    }
    // a wide band: 64 band centroids at a time into a register list
    WaveList<KP> L;
    L.init();
    int nb = 0;
    auto refine = [&](int b0, int n) {
        const bool has = lane < n;
        const int c = band[b0 + (has ? lane : 0)];
        const double dd = exact(c);
        list_offer(L, nprobe, has ? key_of(dd) : kKeyInvalid, has ? c : kIdInvalid);
    };
    if (from_regs) {  // the band is in LDS already
        wave_sync();
#pragma unroll 1
        for (int b0 = 0; b0 < mband; b0 += kWave) refine(b0, min(kWave, mband - b0));
    } else {
        // the band, from the approximations again (L2), R values per lane loaded per round
        constexpr int R = STREAM ? 8 : 1;
        const int nch = (nlist + kWave - 1) / kWave;
#pragma unroll 1
        for (int i0 = 0; i0 < nch; i0 += R) {
            float xs[R];
#pragma unroll
            for (int u = 0; u < R; ++u) {
                const int c = (i0 + u) * kWave + lane;
                xs[u] = c < nlist ? arow[c] : INFINITY;
            }
#pragma unroll 1
            for (int u = 0; u < R; ++u) {
                const int c = (i0 + u) * kWave + lane;
                const bool take = c < nlist && xs[u] <= thr;
                const uint64_t mk = __ballot(take);
                if (take) band[nb + mask_rank(mk)] = c;
                nb += __popcll(mk);
                if (nb >= kWave) {
                    wave_sync();
                    refine(0, kWave);
                    wave_sync();
                    const int rest = nb - kWave;  // <= 63 entries move down
                    const int moved = lane < rest ? band[kWave + lane] : 0;
                    wave_sync();
                    if (lane < rest) band[lane] = moved;
                    wave_sync();
                    nb = rest;
                }
            }
        }
        if (nb > 0) {
            wave_sync();
            refine(0, nb);
        }
    }
    if (lane < nprobe) emit(lane, L.k0, L.i0);
    if constexpr (KP == 128) {
        if (kWave + lane < nprobe) emit(kWave + lane, L.k1, L.i1);
    }
}

#define TRIDENT_SELECT_BAND(KP, V, S)                                                           \
    template __global__ void select_band_kernel<KP, V, S>(                                      \
        const float*, const double*, const float*, const unsigned long long*, double, int, int,  \
        int, int, double, double, const float*, int, int, int32_t*, float*, int, int32_t*, float*, int);
TRIDENT_SELECT_BAND(64, 16, false)
TRIDENT_SELECT_BAND(64, 32, false)
TRIDENT_SELECT_BAND(128, 16, false)
TRIDENT_SELECT_BAND(128, 32, false)
TRIDENT_SELECT_BAND(64, 8, true)
TRIDENT_SELECT_BAND(128, 8, true)
#undef TRIDENT_SELECT_BAND

}  // namespace trident
