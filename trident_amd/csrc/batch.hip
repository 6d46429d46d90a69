// Cluster-batched cascade on the gfx950 int8 matrix cores.
//
// When many queries probe the same cluster (r = B * nprobe / nlist is ~600 at cfg 2), the SQ8
// bound is a dense contraction: codes [n_c x D_pad] (u8) times per-query weights
// [D_pad x queries].  For vector x (codes c_d, cluster vmin/delta) and query q with
// q'_d = q_rot,d - vmin_d and w_d = delta_d * q'_d:
//
//     |x_hat - q_rot|^2 = A_x - 2 sum_d c_d w_d + Q_q,   A_x = sum_d (c_d delta_d)^2,  Q_q = |q'|^2
//
// w is quantised to w = s * w_int + err (s a power of two shared by the <= 32 pairs of a weight
// group, |w_int| <= 32639, split w_int = 256 * hi + lo into two int8 planes); with
// c' = c - 128 the dot product
//     sum_d c_d w_int,d = 256 * MFMA(c', hi) + MFMA(c', lo) + 128 * sum_d w_int,d
// is computed EXACTLY by v_mfma_i32_16x16x64_i8 (two per 64 dims), and
// |sum_d c_d w_d - s * dot| <= 255 * sum_d |w_d - s w_int,d| = err_q.  The triangle inequality
// with r_x >= |x_rot - x_hat| (per vector) and e_q >= |q_rot(float64) - q_rot(exact)| gives
//     lower bound:  |x_rot - q_rot| >= sqrt(A_x + Q_q - 2 s dot - 2 err_q) - r_x - e_q
//     upper bound:  |x_rot - q_rot| <= sqrt(A_x + Q_q - 2 s dot + 2 err_q) + r_x + e_q
// Scaled by the rotation's squared singular-value bounds these bound the canonical float64
// distance.
//
// Pass A (seeding, Stage X; reference src/trident_v4_kernels.cu:626-676): for the seeding
//               probes of each query (the first p_init, or every probe with TRIDENT_UB_SEED 2)
//               every row's upper bound; each unit (<= 16 queries) appends its K smallest
//               (bound, row) entries to the query's list.  ub_kth_kernel then takes the query's
//               K smallest entries (the seeds), refines them exactly and sets
//               tau[q] = min(K-th bound, K-th seed distance); the seeds become the query's
//               first candidates.
// Pass B (LB, Stage Y):  for every probe, rows whose lower bound passes tau[q] are queued in LDS
//               and appended (sorted position) to the query's candidate list.  The test is one
//               int32 compare per (row, query) lane group, max(acc + kq) >= thr_x, with
//               per-query and per-vector constants rounded outward (0.04% of (row, query)
//               pairs survive on cfg-2 data); weight groups without the integer form use a
//               float32 test with an additive slack that bounds every rounding of it.
// Refine (Stage Z, :796-941): one wave per (query, 64-slot chunk of its list) computes the
//               canonical float64 distance of each listed non-seed survivor and keeps it iff
//               <= tau[q].
//
// Scheduling: a work unit is (cluster, a block of its queries, slice of <= ~1024 of its
// vectors).  Pass B (narrow layout, D_pad <= 256): queries are the MFMA's A rows (16 per MFMA,
// two halves = 32 per wave, 128 per unit), vectors its B columns, so a slice's codes are staged
// in LDS once per 128 queries.  Pass A and the wide layout (D_pad > 256): vectors are the A rows
// and 16 queries per wave the B columns.  Units of one launch are split into 8 contiguous
// ranges, one per XCD (blockIdx & 7), so a cluster's codes are read from HBM once per XCD and
// then served by that XCD's L2; within a range each workgroup takes the next unit from its
// XCD's counter (persistent grid, one atomic per unit).  The slice streams through LDS in
// 64-vector blocks (16 in the wide layout), double-buffered: block b + 1 moves global -> LDS
// with direct loads (16-byte code cells, 1 KiB contiguous per wave and load) while the waves
// compute block b, one barrier per block.  Lane l = (i = l & 15, g = l >> 4) holds, for every
// 64-dim step, bytes of dims step*64 + g*16 + [0, 16) of its A row i and of its B column i (any
// dim-to-byte assignment shared by A and B computes the same contraction); the result row
// 4g + r, column i sits in lane l, register r.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace trident {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kUbList = 16;  // per-lane upper-bound list
constexpr int kBlkV = 64;    // slices start on multiples of 64 vectors (whole LDS blocks)
constexpr int kWaveQ = 16;   // queries per wave

// Vector slices of a cluster (both passes), so that no unit runs far longer than the others.
// The seeding pass loses nothing by slicing: every unit hands its K smallest bounds to the
// query's list, and the threshold is the K-th smallest over all of them.
__device__ __forceinline__ int splits_of(int n, int sv) {
    if (n <= 0) return 0;
    return min(kMaxSplit, (n + sv - 1) / sv);
}

// Slices a seeding unit set scans: the first seed_sl of a cluster's slices (sv rows each; the
// caller's choice, 1 or 2).  Seeding needs K good rows per query, not every row of its first
// probes; the threshold stays exact (the K-th exact distance of rows that exist), only looser.
__device__ __forceinline__ int seed_slices(int S, int seed_sl) { return min(S, seed_sl); }

// Entry e < nlist: the seeding units of cluster e (its pass-1 queries, or all of them when
// seed_all, <= 16 per unit; the first seed_slices(S, seed_sl) slices); entry nlist + c: the
// lower-bound units of cluster c (all its queries, <= uqB per unit, every slice).
__device__ __forceinline__ int units_of_entry(const int32_t* seg, const int32_t* vec_off,
                                              int nlist, int uqB, int seed_all, int seed_sl, int sv,
                                              int svb, int e) {
    const int p = e >= nlist ? 1 : 0, c = e - p * nlist;
    const int q = (p || seed_all ? seg[c + 1] : seg[nlist + 1 + c]) - seg[c];
    const int uq = p ? uqB : kUnitQ0;
    const int S = splits_of(vec_off[c + 1] - vec_off[c], p ? svb : sv);
    return q > 0 ? ((q + uq - 1) / uq) * (p ? S : seed_slices(S, seed_sl)) : 0;
}

__device__ __forceinline__ int groups_of_cluster(const int32_t* seg, int c) {
    return (seg[c + 1] - seg[c] + kGroupQ - 1) / kGroupQ;
}

// Exclusive scans of the unit counts of the 2 * nlist (pass, cluster) entries and of the
// weight-group counts of the nlist cluster segments, in two launches of ceil(2 nlist / kBlock)
// <= kBlock blocks, one entry (and one cluster) per thread: in-block offsets plus block totals
// (blk_tot[b] units, blk_tot[kBlock + b] groups), then the carries of the blocks before.
__global__ __launch_bounds__(256) void unit_scan_local_kernel(const int32_t* seg,
                                                              const int32_t* vec_off, int nlist,
                                                              int uqB, int seed_all, int seed_sl,
                                                              int sv, int svb, int32_t* unit_off,
                                                              int32_t* grp_off, int32_t* blk_tot) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t nu =
        i < 2 * nlist ? (uint32_t)units_of_entry(seg, vec_off, nlist, uqB, seed_all, seed_sl, sv, svb, i)
                      : 0u;
    const uint32_t ng = i < nlist ? (uint32_t)groups_of_cluster(seg, i) : 0u;
    uint32_t tu = 0, tg = 0;
    const uint32_t ru = block_exclusive_scan(nu, s_wtot, &tu);
    const uint32_t rg = block_exclusive_scan(ng, s_wtot, &tg);
    if (i < 2 * nlist) unit_off[i] = (int32_t)ru;
    if (i < nlist) grp_off[i] = (int32_t)rg;
    if (threadIdx.x == 0) {
        blk_tot[blockIdx.x] = (int32_t)tu;
        blk_tot[kBlock + blockIdx.x] = (int32_t)tg;
    }
}

__global__ __launch_bounds__(256) void unit_scan_carry_kernel(int nlist, const int32_t* blk_tot,
                                                              int nblk, int32_t* unit_off,
                                                              int32_t* grp_off) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    __shared__ uint32_t s_carry[2];
    const int tid = threadIdx.x, i = blockIdx.x * kBlock + tid;
    uint32_t tu = 0, tg = 0;
    const uint32_t cu = block_exclusive_scan(tid < nblk ? (uint32_t)blk_tot[tid] : 0u, s_wtot, &tu);
    const uint32_t cg =
        block_exclusive_scan(tid < nblk ? (uint32_t)blk_tot[kBlock + tid] : 0u, s_wtot, &tg);
    if (tid == (int)blockIdx.x) {
        s_carry[0] = cu;
        s_carry[1] = cg;
    }
    __syncthreads();
    if (i < 2 * nlist) unit_off[i] += (int32_t)s_carry[0];
    if (i < nlist) grp_off[i] += (int32_t)s_carry[1];
    if (blockIdx.x == 0 && tid == 0) {
        unit_off[2 * nlist] = (int32_t)tu;
        grp_off[nlist] = (int32_t)tg;
    }
}

// Largest e in [0, n) with off[e] <= x (off non-decreasing, off[0] <= x).
__device__ __forceinline__ int seg_search(const int32_t* off, int n, int x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= x) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// One thread per weight group ({first pair, pair count}: kGroupQ consecutive pairs of a cluster's
// segment), then one thread per unit: its segment by binary search over unit_off, then its
// vector slice and query block.  Slices start on 64-vector blocks and are never empty (n > 64 S
// (S - 1) whenever S = ceil(n / sv) > 1, for sv >= 512).
__global__ __launch_bounds__(256) void unit_fill_kernel(const int32_t* seg, const int32_t* vec_off,
                                                        int nlist, int uqB, int seed_all, int sv, int svb,
                                                        const int32_t* unit_off,
                                                        int4* units, int max_units,
                                                        const int32_t* grp_off, int2* groups,
                                                        int max_groups) {
    const int ngrp = min(grp_off[nlist], max_groups);
    for (int gi = blockIdx.x * blockDim.x + threadIdx.x; gi < ngrp;
         gi += gridDim.x * blockDim.x) {
        const int c = seg_search(grp_off, nlist, gi);
        const int k = gi - grp_off[c];
        groups[gi] = make_int2(seg[c] + k * kGroupQ, min(kGroupQ, seg[c + 1] - seg[c] - k * kGroupQ));
    }
    const int E = 2 * nlist;
    const int total = min(unit_off[E], max_units);
    for (int u = blockIdx.x * blockDim.x + threadIdx.x; u < total; u += gridDim.x * blockDim.x) {
        const int e = seg_search(unit_off, E, u);
        const int p = e >= nlist ? 1 : 0, c = e - p * nlist;
        const int n = vec_off[c + 1] - vec_off[c];
        const int S = splits_of(n, p ? svb : sv);
        const int local = u - unit_off[e];
        const int q = (p || seed_all ? seg[c + 1] : seg[nlist + 1 + c]) - seg[c];
        const int uq = p ? uqB : kUnitQ0;
        // slice-major: a slice's query blocks are consecutive units, so the workgroups that
        // take them together read the slice's codes while they are in the XCD's L2
        const int QB = (q + uq - 1) / uq;
        const int sp = local / QB, qb = local - sp * QB;
        const int cnt = min(uq, q - qb * uq);
        const int len = ((n + S - 1) / S + kBlkV - 1) & ~(kBlkV - 1);
        const int vb = sp * len, ve = min(n, vb + len);
        units[u] = make_int4(c | (cnt << 20), seg[c] + qb * uq, vb, ve);
    }
}

__global__ void fill_u64_kernel(unsigned long long* p, unsigned long long v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}


// Fine-level bounds of sorted row pos for a query whose float64 rotated row is q64 (D_pad
// values) and whose rotation error has norm <= qe: lb <= d64(x, q) <= ub.  The row's fine codes
// (16 bits per dimension on its own grid) give x_fine_d = offset + code_d * step, one rounding
// per dimension (the product is exact in float64), as the builder computes it, and
// rho_x >= |x_rot(exact) - x_fine|.  With h = |x_fine - q64| in float64 (relative error
// <= (D_pad + 2) 2^-53 < 1e-12), |x_rot - q_rot| lies in [h (1 - 1e-12) - rho_x - qe,
// h (1 + 1e-12) + rho_x + qe], mapped to the original space by the rotation's squared
// singular-value bounds, with 1e-12 for the canonical float64 distance's own rounding.
__device__ inline void fine_row_bounds(const BatchArgs& a, const double* q64, double qe, int pos,
                                       double& lb, double& ub) {
    const int D_pad = a.D_pad;
    const uint4* rc = reinterpret_cast<const uint4*>(a.fine_codes + (size_t)pos * D_pad);
    const float4 qp = reinterpret_cast<const float4*>(a.fine_qp)[pos];  // offset, step, rho
    const double o = (double)qp.x, st = (double)qp.y;
    double s = 0.0;
    for (int g0 = 0; g0 < D_pad / 8; g0 += 16) {  // 128 dims, sixteen 16-byte loads in flight
        uint4 w[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) w[u] = g0 + u < D_pad / 8 ? rc[g0 + u] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            if (g0 + u >= D_pad / 8) break;
            const uint32_t w4[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const double c = (double)((w4[k >> 1] >> (16 * (k & 1))) & 0xffffu);
                const double t = fma(c, st, o) - q64[8 * (g0 + u) + k];
                s = fma(t, t, s);
            }
        }
    }
    const double h = sqrt(s);
    const double e = (double)qp.z + qe;
    const double lo = fmax(h * (1.0 - 1e-12) - e, 0.0), hi = h * (1.0 + 1e-12) + e;
    lb = lo * lo / a.rot_sq_max * (1.0 - 1e-12);
    ub = hi * hi / a.rot_sq_min * (1.0 + 1e-12);
}

// Fine filter (fine_mode), after the lower-bound pass, in two launches:
//   fine_filter_kernel: the fine-level bounds of every listed survivor, one wave per (query,
//     64-slot chunk) as the refine (a query with many survivors spreads over many waves); the
//     slot's key holds them until the refine: lb rounded down to float32 in the high word, ub
//     rounded up in the low word;
//   fine_tau_kernel: one wave per query, tau drops to the K-th smallest ub (K distinct rows have
//     d64 <= it).
// Every row with d64 <= the old tau is listed, so every row of the exact top-K keeps
// lb <= the new tau, and the refine reads only rows with lb <= tau.  An overflowed list
// (count > cap) is left alone: the merge rescans that query's probes.
__device__ __forceinline__ float fine_lb_of(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }
__device__ __forceinline__ float fine_ub_of(uint64_t k) { return __uint_as_float((uint32_t)k); }

template <int DQ>
__global__ __launch_bounds__(256) void fine_filter_kernel(BatchArgs a, int B) {
    __shared__ double s_q64[kWavesPerBlock][DQ];
    const int lane = threadIdx.x & 63, wid = (int)(threadIdx.x >> 6);
    const int q = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + wid);
    if (q >= B) return;
    const int cnt = a.cand_cnt[q];
    if (cnt > a.cap || (int)blockIdx.y * kWave >= cnt) return;
    for (int d = lane; d < a.D_pad; d += kWave) s_q64[wid][d] = a.xrot64[(size_t)q * a.D_pad + d];
    wave_sync();
    const double qe = sqrt(a.qep[q]) * (1.0 + 1e-12);
    uint64_t* ck = a.cand_key + (size_t)q * a.cap;
    const int32_t* ci = a.cand_id + (size_t)q * a.cap;
    for (int sl = (int)blockIdx.y * kWave + lane; sl < cnt; sl += kWave * (int)gridDim.y) {
        double lb, ub;
        fine_row_bounds(a, s_q64[wid], qe, ci[sl], lb, ub);
        ck[sl] = ((uint64_t)__float_as_uint(__double2float_rd(lb)) << 32) |
                 __float_as_uint(__double2float_ru(ub));
    }
}

// The K-th smallest ub (the low half of a (lb, ub) key) over slots [0, n) of one query's
// candidate list, one wave; +inf when n < K.  The ub are non-negative floats, so their bit
// patterns order as their values.
template <int KP>
__device__ __forceinline__ float listed_kth_ub(const BatchArgs& a, const uint64_t* ck, int n) {
    const int lane = threadIdx.x & 63;
    if (n < a.K) return INFINITY;
    if (n <= 4 * kWave) {
        // Up to 256 slots: bisection on the float32 bits (0xffffffff marks an empty register):
        // the smallest x with count(ub <= x) >= K, 32 halvings of [0, 2^32 - 1].
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sl = i * kWave + lane;
            v[i] = sl < n ? __float_as_uint(fine_ub_of(ck[sl])) : 0xffffffffu;
        }
        uint32_t lo = 0u, hi = 0xfffffffeu;
        while (lo < hi) {
            const uint32_t mid = lo + ((hi - lo) >> 1);
            int c = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) c += __popcll(__ballot(v[i] <= mid));
            if (c >= a.K) hi = mid;
            else lo = mid + 1u;
        }
        return __uint_as_float(lo);
    }
    if (a.K <= 16) {
        // A long list: each lane keeps the 16 smallest ub of its slots (sorted, in registers;
        // the overall K-th smallest is among the lanes' K smallest), then the same bisection
        // over those 64 x 16 values.
        uint32_t v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0xffffffffu;
        for (int s0 = 0; s0 < n; s0 += 4 * kWave) {
            uint32_t x4[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int sl = s0 + u * kWave + lane;
                x4[u] = sl < n ? __float_as_uint(fine_ub_of(ck[sl])) : 0xffffffffu;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t x = x4[u];
                if (__ballot(x < v[15]) == 0ull) continue;
#pragma unroll
                for (int i = 15; i > 0; --i) v[i] = x < v[i - 1] ? v[i - 1] : (x < v[i] ? x : v[i]);
                v[0] = x < v[0] ? x : v[0];
            }
        }
        uint32_t lo = 0u, hi = 0xfffffffeu;
        while (lo < hi) {
            const uint32_t mid = lo + ((hi - lo) >> 1);
            int c = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) c += __popcll(__ballot(v[i] <= mid));
            if (c >= a.K) hi = mid;
            else lo = mid + 1u;
        }
        return __uint_as_float(lo);
    }
    WaveList<KP> L;
    L.init();
    for (int s0 = 0; s0 < n; s0 += kWave) {
        const int sl = s0 + lane;
        const bool in = sl < n;
        list_offer(L, a.K, in ? key_of((double)fine_ub_of(ck[sl])) : kKeyInvalid, in ? sl : kIdInvalid);
    }
    uint64_t kk;
    int32_t ki;
    L.at(a.K - 1, kk, ki);
    return kk != kKeyInvalid ? (float)dist_of(kk) : INFINITY;
}

template <int KP>
__global__ __launch_bounds__(256) void fine_tau_kernel(BatchArgs a, int B) {
    const int lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6));
    if (q >= B) return;
    const int cnt = a.cand_cnt[q];
    if (cnt <= 0 || cnt > a.cap) return;
    const float t = listed_kth_ub<KP>(a, a.cand_key + (size_t)q * a.cap, cnt);
    if (lane == 0 && t < INFINITY) a.tau[q] = fmin(a.tau[q], (double)t);
}

// Mode 10's matrix-core route for K > 16, after its warm-up pass listed every row of the
// queries' first probes: the K-th smallest listed ub (over the first cap entries when the list
// overflowed: any K distinct probed rows with ub <= t make t an upper bound of the K-th
// smallest distance) becomes the query's threshold (ub_best, read by the main pass, and tau),
// and the list is emptied for the main pass, which lists every probe again.
template <int KP>
__global__ __launch_bounds__(256) void cm_seed_kernel(BatchArgs a, int B) {
    const int lane = threadIdx.x & 63;
    const int q = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6));
    if (q >= B) return;
    const int n = min(a.cand_cnt[q], a.cap);
    const float t = n > 0 ? listed_kth_ub<KP>(a, a.cand_key + (size_t)q * a.cap, n) : INFINITY;
    if (lane == 0) {
        if (t < INFINITY) {
            a.ub_best[q] = min(a.ub_best[q], __float_as_uint(t));
            a.tau[q] = fmin(a.tau[q], (double)t);
        }
        a.cand_cnt[q] = 0;
    }
}

template __global__ void fine_filter_kernel<256>(BatchArgs, int);
template __global__ void fine_filter_kernel<1024>(BatchArgs, int);
template __global__ void fine_tau_kernel<64>(BatchArgs, int);
template __global__ void fine_tau_kernel<128>(BatchArgs, int);
template __global__ void cm_seed_kernel<64>(BatchArgs, int);
template __global__ void cm_seed_kernel<128>(BatchArgs, int);

// One thread per (query, sorted position) pair: the fine-level bounds, for bound-rigour tests.
__global__ void fine_bounds_kernel(BatchArgs a, const int32_t* __restrict__ qids,
                                  const int64_t* __restrict__ spos, int n, double* lb,
                                  double* ub) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = qids[i], pos = (int)spos[i];
    double ep = 0.0;
    for (int d = 0; d < a.D_pad; ++d) ep = fma(a.qerr[(size_t)q * a.D_pad + d], a.qerr[(size_t)q * a.D_pad + d], ep);
    fine_row_bounds(a, a.xrot64 + (size_t)q * a.D_pad, sqrt(ep) * (1.0 + 1e-12), pos, lb[i], ub[i]);
}

// Exact test of the listed survivors, in place: slot s >= seed_cnt[q] of query q holds a sorted
// position on entry and (key, original id) on exit, or (kKeyInvalid, kIdInvalid) when the
// canonical float64 distance exceeds tau[q] or the row is one of the query's seeds (slots
// [0, seed_cnt), refined by ub_kth_kernel: their rows are not read again).  One wave per
// (query, 64-slot chunk of its list), one survivor per lane (a query with many survivors
// spreads over many waves); each lane walks its own row in dimension order with 16-byte loads,
// against the query row staged in LDS (DQ >= D floats per wave: 256, or 1024 for the wide
// batched route).  An overflowed list (count > cap) is left alone: the merge rescans that
// query's probes through the SQ8 bounds (merge_kernel).
template <bool HOST, int DQ>
__global__ __launch_bounds__(256) void refine_survivors_kernel(BatchArgs a, int B) {
    __shared__ __align__(16) float s_q[kWavesPerBlock][HOST ? 1 : DQ];  // host: float64 copy below
    const int lane = threadIdx.x & 63, wid = (int)(threadIdx.x >> 6);
    const int q = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + wid);
    if (q >= B) return;
    const int cnt = a.cand_cnt[q], ns = a.seed_cnt[q];
    if (cnt > a.cap || ns + (int)blockIdx.y * kWave >= cnt) return;
    const double tau = a.tau[q];
    const int D = a.D;  // <= DQ (the launch picks DQ from D)
    if constexpr (!HOST) {
        for (int d = lane; d < D; d += kWave) s_q[wid][d] = a.xq[(size_t)q * D + d];
        __builtin_amdgcn_wave_barrier();
    }
    const float* qr = s_q[wid];
    uint64_t* ck = a.cand_key + (size_t)q * a.cap;
    int32_t* ci = a.cand_id + (size_t)q * a.cap;
    // the seeds' original ids: lane k holds seed k (and seed 64 + k)
    const int so0 = lane < ns ? ci[lane] : -1, so1 = lane + kWave < ns ? ci[kWave + lane] : -1;
    auto is_seed = [&](int oid) {
        bool hit = false;
        for (int k = 0; k < min(ns, kWave); ++k) hit |= oid == __builtin_amdgcn_readlane(so0, k);
        for (int k = kWave; k < ns; ++k) hit |= oid == __builtin_amdgcn_readlane(so1, k - kWave);
        return hit;
    };
    const bool vec4 = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(a.xb) & 15) == 0;
    unsigned long long ins = 0;
    if constexpr (HOST) {
        // base in mapped host memory: rows cross PCIe, so the wave's rows are read whole (512
        // contiguous bytes at a time, a group's loads all in flight: refine_rows) and staged
        // through LDS; seed rows are left out of the group
        __shared__ int32_t s_pos[kWavesPerBlock][kWave];
        __shared__ double s_q64[kWavesPerBlock][DQ];
        __shared__ float s_stage[kWavesPerBlock][kStageCh][kWave + 1];
        for (int d = lane; d < D; d += kWave) s_q64[wid][d] = (double)a.xq[(size_t)q * D + d];
        for (int s0 = ns + (int)blockIdx.y * kWave; s0 < cnt; s0 += kWave * (int)gridDim.y) {
            const int s = s0 + lane;
            const bool in = s < cnt;
            const int pos = in ? ci[s] : 0;
            const int oid = in ? a.orig_ids[pos] : -1;
            // fine_mode: rows whose fine lower bound (the slot's key) exceeds tau stay off PCIe
            const bool need = in && !(ns > 0 && is_seed(oid)) &&
                              !(a.fine_mode && (double)fine_lb_of(ck[s]) > tau);
            const uint64_t m = __ballot(need);
            const int nq = __popcll(m), rk = need ? mask_rank(m) : 0;
            if (need) s_pos[wid][rk] = pos;
            wave_sync();
            double acc = 0.0;
            if (nq > 0) acc = refine_rows(a.xb, a.xb8, D, s_pos[wid], nq, s_stage[wid], s_q64[wid]);
            if (a.host_rows && lane == 0 && nq > 0) atomicAdd(a.host_rows, (unsigned long long)nq);
            wave_sync();
            const double d = shfl_f64(acc, rk);
            const bool ok = need && d <= tau;
            if (in) {
                ck[s] = ok ? key_of(d) : kKeyInvalid;
                ci[s] = ok ? oid : kIdInvalid;
            }
            if (a.stats) ins += __popcll(__ballot(ok));
        }
        if (a.stats && lane == 0 && ins)
            atomicAdd(&a.stats[(q % kStatSlots) * 4 + 3], ins);
        return;
    }
    for (int s = ns + (int)blockIdx.y * kWave + lane; s < cnt; s += kWave * (int)gridDim.y) {
        const int pos = ci[s];
        const int oid = a.orig_ids[pos];
        if ((ns > 0 && is_seed(oid)) || (a.fine_mode && (double)fine_lb_of(ck[s]) > tau)) {
            ck[s] = kKeyInvalid;
            ci[s] = kIdInvalid;
            continue;
        }
        const float* xr = a.xb + (size_t)pos * D;
        double acc = 0.0;
        if (vec4) {
            // the row arrives 64 dims at a time, all 16 loads issued before their first use
            int d = 0;
            auto chunk = [&](auto n4c) {
                constexpr int N4 = decltype(n4c)::value;
                float4 xv[N4];
#pragma unroll
                for (int k = 0; k < N4; ++k) xv[k] = *reinterpret_cast<const float4*>(xr + d + 4 * k);
#pragma unroll
                for (int k = 0; k < N4; ++k) {
                    const float4 y = *reinterpret_cast<const float4*>(qr + d + 4 * k);
                    double t = (double)xv[k].x - (double)y.x;
                    acc = fma(t, t, acc);
                    t = (double)xv[k].y - (double)y.y;
                    acc = fma(t, t, acc);
                    t = (double)xv[k].z - (double)y.z;
                    acc = fma(t, t, acc);
                    t = (double)xv[k].w - (double)y.w;
                    acc = fma(t, t, acc);
                }
                d += 4 * N4;
            };
            while (d + 64 <= D) chunk(std::integral_constant<int, 16>{});
            while (d + 4 <= D) chunk(std::integral_constant<int, 1>{});
        } else {
            for (int d = 0; d < D; ++d) {
                const double t = (double)xr[d] - (double)qr[d];
                acc = fma(t, t, acc);
            }
        }
        const bool ok = acc <= tau;
        ck[s] = ok ? key_of(acc) : kKeyInvalid;
        ci[s] = ok ? oid : kIdInvalid;
        if (a.stats) ins += (unsigned long long)ok;
    }
    if (a.stats) {
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) ins += __shfl_xor(ins, o, kWave);
        if (lane == 0 && ins) atomicAdd(&a.stats[(q % kStatSlots) * 4 + 3], ins);
    }
}

template __global__ void refine_survivors_kernel<false, 256>(BatchArgs, int);
template __global__ void refine_survivors_kernel<true, 256>(BatchArgs, int);
template __global__ void refine_survivors_kernel<false, 1024>(BatchArgs, int);
template __global__ void refine_survivors_kernel<true, 1024>(BatchArgs, int);

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) v += shfl_f64(v, lane_id() ^ o);
    return v;
}

__device__ __forceinline__ double sum16_f64(double v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += shfl_f64(v, lane_id() ^ o);
    return v;
}

// Waves [0, ncl): per-cluster bounds of the f32 slack (ncl = nlist, or 0 when the index
// carries them), A_max = 255^2 sum delta^2 (>= A_x,
// codes <= 255) and r_max = max(2 sqrt(sum eps^2), the largest stored r_x) (the first term
// bounds r_x = |a| + |b| <= 2 |a + b| for the non-negative per-dim error terms when eps bounds
// them; the second holds for any eps, e.g. an index built with the reference's 0.5001 delta),
// and r_lo = the smallest stored r_x of the cluster.  Waves [nlist, nlist + B): per-query sum of qerr^2 (the rotation error of q_rot,
// squared).
__global__ __launch_bounds__(256) void aux_bounds_kernel(BatchArgs a, int ncl, int B,
                                                         double* cbound, double* qep,
                                                         int32_t* unit_ctr) {
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    const int D_pad = a.D_pad;
    // the per-launch state of both passes starts here (one launch instead of three fills):
    // work counters, tau = +inf (pass A takes atomicMin), empty survivor lists (pass B)
    if (blockIdx.x == 0 && unit_ctr)
        for (int i = threadIdx.x; i < 2 * 8 * kCtrStride; i += blockDim.x) unit_ctr[i] = 0;
    if (wv < ncl) {
        const size_t off = a.per_cluster ? (size_t)wv * D_pad : 0;
        double dd = 0.0, ee = 0.0;
        for (int d = lane; d < D_pad; d += kWave) {
            const double dl = (double)a.delta[off + d], e = (double)a.eps[off + d];
            dd = fma(dl, dl, dd);
            ee = fma(e, e, ee);
        }
        dd = wave_sum_f64(dd);
        ee = wave_sum_f64(ee);
        float rlo = INFINITY, rhi = 0.0f;
        const int vend = a.vec_off[wv + 1];
        for (int v = a.vec_off[wv] + lane; v < vend; v += 4 * kWave) {  // 4 loads in flight
            float r4[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                r4[u] = v + u * kWave < vend ? a.vec_Ar[v + u * kWave].y : INFINITY;
            rlo = fminf(rlo, fminf(fminf(r4[0], r4[1]), fminf(r4[2], r4[3])));
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (v + u * kWave < vend) rhi = fmaxf(rhi, r4[u]);
        }
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            rlo = fminf(rlo, __shfl_xor(rlo, o, kWave));
            rhi = fmaxf(rhi, __shfl_xor(rhi, o, kWave));
        }
        if (lane == 0) {
            cbound[kCbStride * wv] = 65025.0 * dd * (1.0 + 1e-12);
            cbound[kCbStride * wv + 1] = fmax(2.0 * sqrt(ee), (double)rhi) * (1.0 + 1e-12);
            cbound[kCbStride * wv + 2] = rlo < INFINITY ? (double)rlo : 0.0;
        }
    } else if (wv < ncl + B) {
        const int q = wv - ncl;
        const double* qe = a.qerr + (size_t)q * D_pad;
        double ep = 0.0;
        for (int d = lane; d < D_pad; d += kWave) ep = fma(qe[d], qe[d], ep);
        ep = wave_sum_f64(ep);
        if (lane == 0) {
            qep[q] = ep;
            a.tau[q] = INFINITY;
            a.cand_cnt[q] = 0;
            a.ub_cnt[q] = 0;
            a.ub_best[q] = 0x7f800000u;  // +inf
            a.seed_cnt[q] = 0;
        }
    }
}

// One weight group per wave (its <= 32 pairs share a cluster), 2 lanes per pair: lane l =
// lane % 2 of pair slot lane / 2 owns dims 64 k + 32 l + [0, 32) of every 64-dim step k
// (16-byte loads, two 16-byte stores per plane and step), so the group's scale is a wave
// reduction (no LDS, no barrier) and the per-pair sums take one shuffle.  The queries' int8
// weight planes against the cluster's SQ8 grid and each pair's threshold-independent scalars,
// all in float32 on the float32 rotated query q32 (the bounds take q32 as the query point: e_q
// grows by |q32 - q64| <= 2^-24 |q32| per dimension):
//   w_d = delta_d * (q32_d - vmin_d) (two roundings, <= 2^-22 |w_d|, charged to err_q);  one
//   scale for the group: s = 2^(ilogb(m) - 14), doubled if m / s > 32639, for m = the largest
//   |w_d| of the group's pairs, so |w_int| <= 32639;  w_int = rint(w / s) = 256 hi + lo
//   (hi, lo in [-128, 127]);  Q = sum (q32_d - vmin_d)^2 (relative error < 2^-15).
// The quantisation error is charged by its bound, |w - s w_int| <= s / 2 per dimension:
//   err_q = 255 (D_pad s / 2 + 2^-22 sum |w|),  and |w_int| <= |w| / s + 1 / 2 gives
//   acc_max = 128 (sum |w| / s + D_pad / 2) >= |sum (c - 128) w_int|
// (per-dimension sums of the exact residuals would tighten err_q by ~2x, a 2^-16-relative
// change of the bounds, for four more instructions per dimension).
// (A common scale lets the lower-bound scan compare a wave's 32 queries against one integer
// threshold per vector.)  Plane bytes past D_pad (up to DP) are zero, so the scan may read
// whole 64-dim steps.
template <int KS>
__global__ __launch_bounds__(256) void pair_prep_kernel(BatchArgs a) {
    const int lane = threadIdx.x & 63, l = lane & 1, slot = lane >> 1;
    const int gi = blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    if (gi >= min(a.grp_off[a.nlist], a.max_groups)) return;
    const int2 grp = a.groups[gi];
    const bool valid = slot < grp.y;
    const int pp = grp.x + (valid ? slot : 0);  // idle slots redo the first pair, store nothing
    const int c = a.pair_cid[pp], q = a.pair_qid[pp];
    const int D_pad = a.D_pad, DP = a.DP;
    const size_t off = a.per_cluster ? (size_t)c * D_pad : 0;
    const float* xr = a.xrot32 + (size_t)q * D_pad;
    // Up to 128 dims the weights stay in registers between the group scale and the
    // quantisation; wider, the second loop recomputes them (the same operations, so the same
    // values).
    constexpr bool KEEP = KS <= 2;
    float w[KEEP ? KS : 1][32];
    float mx = 0.0f, Qp = 0.0f, qq = 0.0f, wl1 = 0.0f;
    auto weights = [&](int k, float (&wk)[32], auto sums_c) {
        constexpr bool SUMS = decltype(sums_c)::value;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int d0 = 64 * k + 32 * l + 16 * h2;  // D_pad is a multiple of 32: all 16 or none
#pragma unroll
            for (int e = 0; e < 16; ++e) wk[16 * h2 + e] = 0.0f;
            if (d0 < D_pad) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float4 x4 = *reinterpret_cast<const float4*>(xr + d0 + 4 * h);
                    const float4 v4 = *reinterpret_cast<const float4*>(a.vmin + off + d0 + 4 * h);
                    const float4 g4 = *reinterpret_cast<const float4*>(a.delta + off + d0 + 4 * h);
                    const float xv[4] = {x4.x, x4.y, x4.z, x4.w}, vv[4] = {v4.x, v4.y, v4.z, v4.w},
                                gv[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float qp = xv[e] - vv[e];
                        wk[16 * h2 + 4 * h + e] = gv[e] * qp;
                        if constexpr (SUMS) {
                            mx = fmaxf(mx, fabsf(wk[16 * h2 + 4 * h + e]));
                            wl1 += fabsf(wk[16 * h2 + 4 * h + e]);
                            Qp = fmaf(qp, qp, Qp);
                            qq = fmaf(xv[e], xv[e], qq);
                        }
                    }
                }
            }
        }
    };
    if constexpr (KEEP) {
#pragma unroll
        for (int k = 0; k < KS; ++k) weights(k, w[k], std::true_type{});
    } else {
        // rolled loops: unrolled, the compiler would keep every step's weights live into the
        // second loop instead of recomputing them
#pragma unroll 1
        for (int k = 0; k < KS; ++k) {
            float wk[32];
            weights(k, wk, std::true_type{});
        }
    }
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));  // the group
    // the pair's two lanes
    Qp += __shfl_xor(Qp, 1, kWave);
    qq += __shfl_xor(qq, 1, kWave);
    wl1 += __shfl_xor(wl1, 1, kWave);
    float l1g = wl1;  // the group's largest sum |w|
#pragma unroll
    for (int o = 2; o < kWave; o <<= 1) l1g = fmaxf(l1g, __shfl_xor(l1g, o, kWave));
    // s and 1/s are powers of two in [2^-114, 2^114], so w * (1/s) is exactly w / s and
    // s * wi is exact.  Two limits: |w_int| <= 32639 (the hi / lo split), and, for every pair,
    // sum |w_int| <= sum |w| / s + D_pad / 2 <= 2^23 - 1, so that |acc| <= 128 sum |w_int| <
    // 2^30 and the lower-bound test's acc + kq (|kq| <= 2^30) stays inside int32.  The second
    // follows from the first while D_pad <= 256; it binds only for wider weights.
    int es = 0;
    if (mx > 0x1p-100f) {
        es = ilogbf(mx) - 14;
        if (ldexpf(mx, -es) > 32639.0f) ++es;
        const float lim = 8388607.0f - 0.5f * (float)D_pad;
        const float l1u = l1g * (1.0f + (float)a.sum_rel);
        for (int i = 0; i < 8 && ldexpf(l1u, -es) > lim; ++i) ++es;
    }
    const float s = ldexpf(1.0f, es), inv_s = ldexpf(1.0f, -es);
    int wsum = 0, lsum = 0, lsq = 0;  // sum w_int, sum |lo|, sum lo^2 (<= 2^14 DP)
    int8_t* hi_p = a.pw + (size_t)pp * 2 * DP;
#pragma unroll KEEP ? KS : 1
    for (int k = 0; k < KS; ++k) {
        float wre[32];
        if constexpr (!KEEP) weights(k, wre, std::false_type{});
        const float(&wk)[32] = KEEP ? w[KEEP ? k : 0] : wre;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                int wi[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wi[e] = (int)rintf(wk[16 * h2 + 4 * h + e] * inv_s);  // 0 for dims >= D_pad
                    wsum += wi[e];
                    const int lo = (int)(int8_t)(wi[e] & 0xff);
                    lsum += abs(lo);
                    lsq += lo * lo;
                }
                // lo = the low byte of wi as int8, hi = (wi - lo) / 256 = the second byte of
                // wi + 128
                lw[h] = ((uint32_t)wi[0] & 0xffu) | (((uint32_t)wi[1] & 0xffu) << 8) |
                        (((uint32_t)wi[2] & 0xffu) << 16) | ((uint32_t)wi[3] << 24);
                hw[h] = (((uint32_t)(wi[0] + 128) >> 8) & 0xffu) |
                        ((uint32_t)(wi[1] + 128) & 0xff00u) |
                        ((((uint32_t)(wi[2] + 128) >> 8) & 0xffu) << 16) |
                        ((uint32_t)(wi[3] + 128) >> 8 << 24);
            }
            if (valid) {
                const int b = 64 * k + 32 * l + 16 * h2;
                *reinterpret_cast<uint4*>(hi_p + b) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                *reinterpret_cast<uint4*>(hi_p + DP + b) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            }
        }
    }
    wsum += __shfl_xor(wsum, 1, kWave);
    lsum += __shfl_xor(lsum, 1, kWave);
    lsq += __shfl_xor(lsq, 1, kWave);
    if (valid && l == 0) {
        PairRec r;
        r.Qp = (double)Qp;
        // float32 sums of D_pad non-negative terms: relative error < sum_rel (the
        // (1 + sum_rel) factors here and the sum_rel margins on Qp where it is used)
        const double l1 = (double)wl1 * (1.0 + a.sum_rel);
        r.err_q = 255.0 * (0.5 * (double)D_pad * (double)s + 0x1p-22 * l1);
        // the query is the float32 rotation q32: |q32 - q_exact| <= e_q(float64) + 2^-23 |q32|
        r.e_q = sqrt(a.qep[q]) * (1.0 + 1e-12) + 0x1p-23 * sqrt((double)qq) * (1.0 + a.sum_rel) +
                1e-30;
        r.cW = 128.0 * (double)wsum;
        r.c1 = 2.0 * (double)s;
        r.a_max = a.cbound[kCbStride * c];
        r.r_max = a.cbound[kCbStride * c + 1];
        r.acc_max = 128.0 * (l1 * (double)inv_s + 0.5 * (double)D_pad);
        r.lo_max = 128.0 * (double)lsum;  // <= 128 * 128 * D_pad <= 2^24
        r.lo_l2 = sqrt((double)lsq) * (1.0 + 0x1p-50);  // lsq is exact; sqrt within half an ulp
        a.prec[pp] = r;
    }
}

template __global__ void pair_prep_kernel<1>(BatchArgs);
template __global__ void pair_prep_kernel<2>(BatchArgs);
template __global__ void pair_prep_kernel<3>(BatchArgs);
template __global__ void pair_prep_kernel<4>(BatchArgs);
template __global__ void pair_prep_kernel<5>(BatchArgs);
template __global__ void pair_prep_kernel<6>(BatchArgs);
template __global__ void pair_prep_kernel<7>(BatchArgs);
template __global__ void pair_prep_kernel<8>(BatchArgs);
template __global__ void pair_prep_kernel<9>(BatchArgs);
template __global__ void pair_prep_kernel<10>(BatchArgs);
template __global__ void pair_prep_kernel<11>(BatchArgs);
template __global__ void pair_prep_kernel<12>(BatchArgs);
template __global__ void pair_prep_kernel<13>(BatchArgs);
template __global__ void pair_prep_kernel<14>(BatchArgs);
template __global__ void pair_prep_kernel<15>(BatchArgs);
template __global__ void pair_prep_kernel<16>(BatchArgs);

// m <- the 16 smallest of two ascending 16-lists (m, o), ascending, all in registers:
// min(m[i], o[15 - i]) is a bitonic sequence holding them; four half-cleaner stages sort it.
__device__ __forceinline__ void merge16(float (&m)[16], const float (&o)[16]) {
    float c[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = fminf(m[i], o[15 - i]);
#pragma unroll
    for (int d = 8; d >= 1; d >>= 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if ((i & d) == 0) {
                const float lo = fminf(c[i], c[i + d]), hi = fmaxf(c[i], c[i + d]);
                c[i] = lo;
                c[i + d] = hi;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) m[i] = c[i];
}

// Merge the lists of lanes l, l ^ 16, l ^ 32, l ^ 48 (one query's four lane groups).
__device__ __forceinline__ void merge16_groups(float (&m)[16]) {
#pragma unroll
    for (int o = 16; o < kWave; o <<= 1) {
        float other[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) other[i] = __shfl_xor(m[i], o, kWave);
        merge16(m, other);
    }
}

// Residual-norm band (reference src/trident_v4_kernels.cu:686-695): |q - x| >= | |q - c| -
// |x - c| |, so no vector of a tile whose |x - c| lies in [rmin, rmax] is within sqrt(tau) of q
// when rmax < dqc - sqrt(tau) or rmin > dqc + sqrt(tau).  tol covers the float32 storage of
// both norms (as the per-pair route).  A query without a threshold never skips.
__device__ __forceinline__ bool l1_skips(float dqc, double tau, float rmin, float rmax) {
    if (!(tau < (double)INFINITY)) return false;
    const double t = sqrt(tau) * (1.0 + 1e-6), dq = (double)dqc, rmx = (double)rmax;
    const double tol = 1e-6 * (dq + rmx) + 1e-30;
    return rmx + tol < dq - t || (double)rmin - tol > dq + t;
}

// Integer lower-bound threshold of one vector for a wave: an int32 <= (A - r (r + 2 tq)) / c1
// for the stored A (rounded down), r and tq (rounded up), computed in f32 with a margin m of
// 2^-21 (A + y) / c1 + 1 over its three roundings (each <= 2^-24 of a term <= A + y); c1 is a
// power of two, so the scaling is exact.  Out-of-range values saturate to [-2^31 + 128,
// 2^31 - 128] (a NaN from an overflowed margin gives the lower end: every row passes); rows past
// the slice (r = +inf) get INT_MAX.  The tested sum S = acc + kq of a real query lies in
// [-2^31 + 128, 2^31 - 128] (|acc| <= 128 (2^23 - 1), |kq| <= 2^30), so the lower clamp never
// rejects a row the exact threshold passes, rows past the slice never pass, and an empty query
// row (zero weights, kq = INT_MIN) never passes either.
__device__ __forceinline__ int lb_thr(float A, float r, float tq, float inv_c1) {
    const float y = r * fmaf(2.0f, tq, r);
    const float X = (A - y) * inv_c1;
    const float m = fmaf(0x1p-21f * (A + y), inv_c1, 1.0f);
    const float v = fminf(fmaxf(floorf(X - m), -2147483520.0f), 2147483520.0f);
    return r <= 3.0e38f ? (int)v : INT_MAX;
}

// Global -> LDS without registers: lane i's 16 (or 4) bytes, read from base + off (base
// wave-uniform, off per lane), land at lds + 16 i (4 i).  Written as inline asm on purpose:
// the compiler tracks its own direct loads by LDS object and, when it cannot tell two halves
// of one array apart, makes every LDS read wait for all loads in flight, which stalls each
// block's first tile on the next block's loads.  It does not see these, so the callers wait
// themselves (vmcnt(0) before the barrier that publishes a block); the compiler's waits for
// its own global loads only grow more conservative (the counter retires in order).
// A generic pointer into LDS is the shared aperture's base in the high half and the LDS
// address in the low half, so the low half is taken as is (an address-space cast would add a
// null test per load).
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(size_t)p; }
// M0 (the LDS address of the load, latched at issue) is saved and restored around it.
// A wave-uniform base pointer kept in SGPRs: inside lane-divergent branches the compiler may
// otherwise materialise it in VGPRs, which the direct loads' saddr operand cannot take.
__device__ __forceinline__ const void* sgpr_ptr(const void* p) {
    const uint64_t v = (uint64_t)(size_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (const void*)(size_t)(((uint64_t)hi << 32) | lo);
}
// Both are wave-uniform at every call; readfirstlane states it, so that the compiler keeps them in
// SGPRs even where it cannot prove the uniformity itself.
__device__ __forceinline__ void load_lds16(const void* base, uint32_t off, const void* lds) {
    uint32_t keep;
    const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr(lds));
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(keep) : "v"(off), "s"(sgpr_ptr(base)), "s"(m) : "memory");
}
__device__ __forceinline__ void load_lds4(const void* base, uint32_t off, const void* lds) {
    uint32_t keep;
    const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr(lds));
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(keep) : "v"(off), "s"(sgpr_ptr(base)), "s"(m) : "memory");
}

// Vectors per LDS block of the scan kernels: 64 while D_pad <= 256 (16 KiB of codes a block),
// 16 for D_pad up to 1024 (at most 16 KiB a block, so two blocks and four waves' weights in
// registers still leave room for several workgroups per CU).
__host__ __device__ constexpr int block_vectors(int KS) { return KS <= 4 ? 64 : 16; }

// Wide layout: blocks in flight ahead of the one being scanned (a ring of kWideAhead + 1 code
// buffers).  With ~200 VGPRs a CU holds two workgroups, so one block in flight each leaves the
// loop waiting on load latency; the row scalars use a ring of 8 (the deferred replica finish
// reads the previous block's).
constexpr int kWideAhead = 2;

// s_waitcnt vmcnt(n) for a wave-uniform n (the count is an instruction immediate); counts
// above 15 wait for everything.
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
#define TRIDENT_VMCNT_CASE(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        TRIDENT_VMCNT_CASE(1) TRIDENT_VMCNT_CASE(2) TRIDENT_VMCNT_CASE(3) TRIDENT_VMCNT_CASE(4)
        TRIDENT_VMCNT_CASE(5) TRIDENT_VMCNT_CASE(6) TRIDENT_VMCNT_CASE(7) TRIDENT_VMCNT_CASE(8)
        TRIDENT_VMCNT_CASE(9) TRIDENT_VMCNT_CASE(10) TRIDENT_VMCNT_CASE(11)
        TRIDENT_VMCNT_CASE(12) TRIDENT_VMCNT_CASE(13) TRIDENT_VMCNT_CASE(14)
        TRIDENT_VMCNT_CASE(15)
#undef TRIDENT_VMCNT_CASE
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// Direct loads of one 16-vector block (the wide layout, D_pad > 256) of code cells -- one
// contiguous run [g][16] of 16-byte cells, g < G16 = D_pad / 16, in the block-major sq8_cells
// -- into an LDS buffer of the same layout, plus the block's row scalars (A_lo, r) into sA /
// sr.  One wave-load moves 1 KiB = 4 groups (one 64-dim step); the workgroup's waves take
// every 4th step.  Groups past G16 (the last step when D_pad is an odd multiple of 32) are not
// loaded: their weights are zero.  Rows past the slice read the slice's last row (never used).
template <int KS>
__device__ __forceinline__ void load_code_block16(const uint4* block_cells, int G16, int wid,
                                                  int lane, uint4* lds, const float2* rows_Ar,
                                                  int row0, int row_last, float* sA,
                                                  float* sr) {
    const uint4* base = static_cast<const uint4*>(sgpr_ptr(block_cells));
#pragma unroll
    for (int jj = 0; jj < (KS + kWavesPerBlock - 1) / kWavesPerBlock; ++jj) {
        const int L = wid + kWavesPerBlock * jj;
        if (L < KS && 4 * L + (lane >> 4) < G16)
            load_lds16(base, 16u * (uint32_t)(L * kWave + lane), lds + L * kWave);
    }
    if (wid == 0 && lane < 16) {
        const void* rb = sgpr_ptr(rows_Ar);
        const uint32_t off = 8u * (uint32_t)min(row0 + lane, row_last);
        load_lds4(rb, off, sA);
        load_lds4(rb, off + 4u, sr);
    }
}

// A seeding bound with its row (index in the unit's slice) in the low 16 bits: rounded up to a
// multiple of 2^16 in the bit pattern first, so it stays an upper bound (at most 2^-7 larger);
// rows past 2^16 - 2 of a slice carry kNoRow.  Non-finite and huge bounds become +inf.
__device__ __forceinline__ float enc_row(float u, int idx) {
    const uint32_t b = __float_as_uint(u);
    if (!(b < 0x7f7f0000u)) return INFINITY;
    const uint32_t r = idx < (int)kNoRow ? (uint32_t)idx : kNoRow;
    return __uint_as_float(((b + 0x10000u) & 0xffff0000u) | r);
}
// The list entry of an encoded bound: (bits, sorted position or -1).
__device__ __forceinline__ uint2 row_entry(float u, int row0) {
    const uint32_t b = __float_as_uint(u), r = b & 0xffffu;
    return make_uint2(b, (u < INFINITY && r != kNoRow) ? (uint32_t)(row0 + (int)r) : 0xffffffffu);
}

// Pass A (seeding), the first p_init probes: for every query of a unit the K-th smallest upper
// bound over the cluster -> atomicMin into tau[q] (float64 bit pattern).  Units (<= 16
// queries, whole clusters) and wave mapping as in lb_scan_kernel; block b + 1's code cells and
// row scalars (A_lo, r) move global -> LDS directly while the waves scan block b.
//
// Per row, in float32, with the per-query constants of the unit prologue:
//     E = fma(-c1, float(acc), Cq) + A_lo (1 + 2^-21),   Cq >= A Q-part - c1 cW + slack,
//     u = fma(sqrt(max(E, 0)), 1 + 2^-20, r + e_q) (1 + 2^-21)  >=  |x_rot - q_rot|,
// where the exact E = A + Q + 2 err - c1 (acc + cW) (norm form of the upper bound) and the
// slack 2^-22 (A_max + c1 acc_max + |Cq|) covers the roundings of float(acc), the fma and the
// add (each <= 2^-24 of a term bounded by that sum); the (1 + 2^-20) factor covers the
// square root's error and (1 + 2^-21) the last two roundings (all terms non-negative).  The
// root is the hardware's v_sqrt_f32 (not the correctly rounded library sequence, 3x the
// instructions): its error, measured over every mantissa of both exponent parities at several
// scales, is at most 0.93 ulp, well inside the 8 ulp that 2^-20 allows; E is raised to at least
// 2^-126 first, so it never sees a denormal (a larger E only raises the bound).  A_lo (1 + 2^-21)
// >= A: vec_Ar holds A rounded down by 1e-13 and then to float32.
//
// Each lane keeps the M smallest bounds of its rows (M = 4 when K <= 16: a query's rows are
// spread over 16 lanes, and the merged lists' K-th entry is the exact K-th smallest unless one
// lane held more than M of them, in which case it is still an upper bound of it).
template <int KS, int M>
__global__ __launch_bounds__(256) void ub_scan_kernel(BatchArgs a) {
    // The code buffers double as the end-of-unit list exchange (after a barrier).
    constexpr int BV = block_vectors(KS);
    constexpr int NBC = BV == 64 ? 2 : kWideAhead + 1;  // code buffers
    constexpr int kCodeU4 = NBC * KS * 4 * BV, kUblU4 = kWavesPerBlock * kWaveQ * kWave / 4;
    __shared__ uint4 s_big[kCodeU4 > kUblU4 ? kCodeU4 : kUblU4];
    uint4(*s_codes)[KS * 4 * BV] = reinterpret_cast<uint4(*)[KS * 4 * BV]>(s_big);
    float(*s_ubl)[kWaveQ * kWave] = reinterpret_cast<float(*)[kWaveQ * kWave]>(s_big);
    // Row scalars: double-buffered with the codes, or (wide layout) a ring of 8 that also
    // holds the block its replica waves finish one block late.  s_part: the replicas' partial
    // sums.
    constexpr int NAB = BV == 64 ? 2 : 8, NP = BV == 64 ? 1 : 2;
    __shared__ __align__(16) float s_A[NAB][BV];
    __shared__ __align__(16) float s_r[NAB][BV];
    __shared__ int4 s_part[NP][NP > 1 ? kWavesPerBlock : 1][NP > 1 ? kWave : 1];
    __shared__ int s_unit[2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int u0 = a.unit_off[a.unit_beg], u1 = min(a.unit_off[a.unit_end], a.max_units);
    const int nx = (max(u1 - u0, 0) + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int rb = u0 + xcd * nx, re = min(u1, rb + nx);
    int32_t* ctr = a.ctr + xcd * kCtrStride;
    const int T = a.T, G16 = a.D_pad >> 4;

    // next unit index: as in lb_scan_kernel
    if (tid == 0) s_unit[0] = atomicAdd(ctr, 1);
    for (int it = 0;; ++it) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + rb;
        if (ui < rb || ui >= re) break;
        int nxt = 0;
        const int4 un = a.units[ui];
        const int cid = un.x & 0xfffff, cnt = un.x >> 20, start = un.y, vb = un.z, ve = un.w;
        const int G = (cnt + kWaveQ - 1) / kWaveQ;
        const int R = kWavesPerBlock / G;
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(kWaveQ, cnt - gq * kWaveQ) : 0;
        const bool hasq = j < nq;
        const int v0 = a.vec_off[cid];
        const int t0 = a.tile_off[cid];

        // ---- this wave's queries: weight planes and float32 bound constants ----
        v4i bhi[KS], blo[KS];
        int q = 0;
        float nc1 = 0.0f, Cq = INFINITY, e_q = 0.0f;  // lanes without a query: u = +inf
        if (active) {
            const int pj = start + gq * kWaveQ + (hasq ? j : 0);
            q = a.pair_qid[pj];
            const int8_t* hp = a.pw + (size_t)pj * 2 * a.DP + g * 16;
            if (BV == 64 || R == 1) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    bhi[ks] = *reinterpret_cast<const v4i*>(hp + ks * 64);
                    blo[ks] = *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64);
                }
            } else {
                // wide layout with R replicas: slot i holds step rr + i R (zero past KS)
#pragma unroll
                for (int i = 0; i < KS; ++i) {
                    const int ks = rr + i * R;
                    bhi[i] = ks < KS ? *reinterpret_cast<const v4i*>(hp + ks * 64) : v4i{0, 0, 0, 0};
                    blo[i] = ks < KS ? *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64)
                                     : v4i{0, 0, 0, 0};
                }
            }
            if (hasq) {
                const PairRec pr = a.prec[pj];
                const double AQ = (pr.Qp * (1.0 + a.sum_rel) + 1e-30 + 2.0 * pr.err_q) * (1.0 + 1e-13);
                const double C = AQ - pr.c1 * pr.cW;
                const double slack =
                    0x1p-22 * (pr.a_max * (1.0 + 0x1p-20) + pr.c1 * pr.acc_max + fabs(C)) *
                        (1.0 + 1e-6) + 1e-30;
                nc1 = -(float)pr.c1;  // a power of two: exact
                Cq = __double2float_ru(C + slack);
                e_q = __double2float_ru(pr.e_q);
            }
        }

        float ubl[kUbList];
#pragma unroll
        for (int i = 0; i < kUbList; ++i) ubl[i] = INFINITY;

        // ---- one 16-vector tile ----
        auto tile = [&](int buf, int t, int li0) {
            const uint4* blk = s_codes[buf];
            v4i A[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 v = blk[(ks * 4 + g) * BV + t * 16 + j];
                A[ks] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
            const int row0 = t * 16 + 4 * g;
            const float4 A4 = *reinterpret_cast<const float4*>(&s_A[buf][row0]);
            const float4 r4 = *reinterpret_cast<const float4*>(&s_r[buf][row0]);
            v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks], bhi[ks], acc_hi, 0, 0, 0);
                acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks], blo[ks], acc_lo, 0, 0, 0);
            }
            const float Av[4] = {A4.x, A4.y, A4.z, A4.w}, rv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int S = (acc_hi[r] << 8) + acc_lo[r];
                const float E = fmaf(nc1, (float)S, Cq) + Av[r] * (1.0f + 0x1p-21f);
                float u = fmaf(__builtin_amdgcn_sqrtf(fmaxf(E, 0x1p-126f)), 1.0f + 0x1p-20f,
                               rv[r] + e_q) * (1.0f + 0x1p-21f);
                u = li0 + 4 * g + r < ve ? enc_row(u, li0 + 4 * g + r - vb) : INFINITY;
                // sorted insertion (selects, not fminf: no NaN here, and no canonicalisation)
                if constexpr (M <= 4) {
#pragma unroll
                    for (int i = M - 1; i > 0; --i)
                        ubl[i] = (u < ubl[i - 1]) ? ubl[i - 1] : (u < ubl[i] ? u : ubl[i]);
                    ubl[0] = u < ubl[0] ? u : ubl[0];
                } else if (u < ubl[M - 1]) {
#pragma unroll
                    for (int i = M - 1; i > 0; --i)
                        ubl[i] = (u < ubl[i - 1]) ? ubl[i - 1] : (u < ubl[i] ? u : ubl[i]);
                    ubl[0] = u < ubl[0] ? u : ubl[0];
                }
            }
        };

        // ---- wide layout (D_pad > 256, one 16-vector tile per block): this wave's share of
        // the 64-dim steps (all of them, or steps rr, rr + R, ... when R replica waves share
        // the tile: each replica's partial sum is exact in int32 like the whole; R is 1, 2 or
        // 4 and a compile-time constant here, so the weight slots stay in registers) ----
        auto wide_partial = [&](int buf, int (&S)[4], auto r_c) {
            constexpr int RC = decltype(r_c)::value, NS = (KS + RC - 1) / RC;
            const uint4* blk = s_codes[buf];
            // every A operand of the wave's steps first (its weight slots past KS are zero, so
            // a clamped step contributes nothing), then the MFMA chains
            v4i A[NS];
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const int ks = RC == 1 ? i : min(rr + i * RC, KS - 1);
                const uint4 v = blk[(ks * 4 + g) * BV + j];
                A[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
            v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], bhi[i], acc_hi, 0, 0, 0);
                acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], blo[i], acc_lo, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) S[r] = (acc_hi[r] << 8) + acc_lo[r];
        };
        // the block's rows from whole sums (rows 4 g + r of the tile, query column j)
        auto wide_rows = [&](const int (&S)[4], int abuf, int li0) {
            const float4 A4 = *reinterpret_cast<const float4*>(&s_A[abuf][4 * g]);
            const float4 r4 = *reinterpret_cast<const float4*>(&s_r[abuf][4 * g]);
            const float Av[4] = {A4.x, A4.y, A4.z, A4.w}, rv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float E = fmaf(nc1, (float)S[r], Cq) + Av[r] * (1.0f + 0x1p-21f);
                float u = fmaf(__builtin_amdgcn_sqrtf(fmaxf(E, 0x1p-126f)), 1.0f + 0x1p-20f,
                               rv[r] + e_q) * (1.0f + 0x1p-21f);
                u = li0 + 4 * g + r < ve ? enc_row(u, li0 + 4 * g + r - vb) : INFINITY;
                if (u < ubl[M - 1]) {
#pragma unroll
                    for (int i = M - 1; i > 0; --i)
                        ubl[i] = (u < ubl[i - 1]) ? ubl[i - 1] : (u < ubl[i] ? u : ubl[i]);
                    ubl[0] = u < ubl[0] ? u : ubl[0];
                }
            }
        };
        // replica (b mod R) of the group finishes block b from the R partial sums
        auto wide_finish = [&](int b, int abuf) {
            if (((b & (R - 1)) != rr)) return;
            int S[4] = {0, 0, 0, 0};
            for (int r2 = 0; r2 < R; ++r2) {
                const int4 p = s_part[b & 1][gq * R + r2][lane];
                S[0] += p.x;
                S[1] += p.y;
                S[2] += p.z;
                S[3] += p.w;
            }
            wide_rows(S, abuf, vb + b * BV);
        };

        // ---- stream the cluster through LDS in 64-vector blocks ----
        const uint4* cells_c = a.cells + (size_t)t0 * G16 * T;
        int ct = vb / T, cw = vb - ct * T;
        auto gload = [&](int buf, int abuf, int blk0) {
            if constexpr (BV == 64) {
                // block-major cells: the block's groups are consecutive runs of 64 cells
                const uint4* base = cells_c + (size_t)ct * G16 * T + (size_t)cw * G16 + wid * BV;
#pragma unroll
                for (int jj = 0; jj < KS; ++jj)
                    if (wid + 4 * jj < G16)
                        load_lds16(base + (size_t)(4 * jj) * BV, 16u * lane,
                                   &s_codes[buf][(wid + 4 * jj) * BV]);
                if (wid == 0) {  // rows past the slice read the slice's last row (never used)
                    const uint32_t off = 8u * (uint32_t)min(blk0 + lane, ve - 1);
                    load_lds4(a.vec_Ar + v0, off, s_A[abuf]);
                    load_lds4(a.vec_Ar + v0, off + 4u, s_r[abuf]);
                }
            } else {
                load_code_block16<KS>(cells_c + (size_t)ct * G16 * T + (size_t)cw * G16, G16,
                                      wid, lane, s_codes[buf], a.vec_Ar + v0, blk0, ve - 1,
                                      s_A[abuf], s_r[abuf]);
            }
            cw += BV;
            if (cw == T) {
                cw = 0;
                ++ct;
            }
        };
        const int nblk = (ve - vb + BV - 1) / BV;
        if constexpr (BV == 64) {
            if (nblk > 0) gload(0, 0, vb);
            for (int b = 0; b < nblk; ++b) {
                const int buf = b & 1;
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                if (tid == 0 && b == max(nblk - 2, 0)) nxt = atomicAdd(ctr, 1);
                const int blk0 = vb + b * BV;
                if (b + 1 < nblk) gload(buf ^ 1, buf ^ 1, blk0 + BV);
                if (active) {
                    for (int t = rr; t < BV / 16; t += R) {
                        if (blk0 + t * 16 >= ve) break;
                        tile(buf, t, blk0 + t * 16);
                    }
                }
            }
        } else {
            // Ring: block b in code buffer b % NBC and row-scalar slot b % 8, with blocks b + 1 ..
            // b + kWideAhead in flight.  A wave waits only for its own loads of block b: the
            // nload per block it issued later may still be outstanding (vector memory
            // operations retire in issue order).  Replicas (R > 1) leave their partial sums of
            // block b in s_part[b & 1]; after the next barrier replica (b mod R) adds them and
            // finishes the rows.
            const int nload = (KS - wid + 3) / 4 + (wid == 0 ? 2 : 0);
            for (int p = 0; p < kWideAhead && p < nblk; ++p) gload(p, p, vb + p * BV);
            int cs = 0;  // b % NBC
            for (int b = 0; b < nblk; ++b) {
                wait_vmcnt(min(kWideAhead - 1, nblk - 1 - b) * nload);
                __syncthreads();
                if (tid == 0 && b == max(nblk - 2, 0)) nxt = atomicAdd(ctr, 1);
                const int blk0 = vb + b * BV;
                if (b + kWideAhead < nblk)  // into the buffer block b - 1 used
                    gload(cs == 0 ? NBC - 1 : cs - 1, (b + kWideAhead) & 7,
                          blk0 + kWideAhead * BV);
                if (active) {
                    int S[4];
                    if (R == 1) {
                        wide_partial(cs, S, std::integral_constant<int, 1>{});
                        wide_rows(S, b & 7, blk0);
                    } else {
                        if (R == 2) wide_partial(cs, S, std::integral_constant<int, 2>{});
                        else wide_partial(cs, S, std::integral_constant<int, 4>{});
                        s_part[b & 1][wid][lane] = make_int4(S[0], S[1], S[2], S[3]);
                        if (b > 0) wide_finish(b - 1, (b - 1) & 7);
                    }
                }
                cs = cs + 1 == NBC ? 0 : cs + 1;
            }
            if (R > 1 && nblk > 0) {
                __syncthreads();
                if (active) wide_finish(nblk - 1, (nblk - 1) & 7);
            }
        }

        // ---- K-th smallest upper bound per query -> atomicMin into tau[q] ----
        //  K <= 16: the four lane groups' lists are merged in registers (exact top 16 of the
        //    kept bounds), replica waves exchange theirs through LDS and the group's first
        //    wave merges them the same way.
        //  K > 16: all R x 64 lists go through a register bitonic list.
        // Either way the K-th entry is an upper bound of the K-th smallest distance bound.
        __syncthreads();  // every wave is done with the code buffers
        if (a.K <= kUbList) {
            if (active) {
                merge16_groups(ubl);
                if (R > 1 && g == 0) {
#pragma unroll
                    for (int i = 0; i < kUbList; ++i) s_ubl[wid][j * kUbList + i] = ubl[i];
                }
            }
            if (R > 1) {
                __syncthreads();
                if (active && rr == 0) {
#pragma unroll
                    for (int i = 0; i < kUbList; ++i)
                        ubl[i] = g < R ? s_ubl[wid + g][j * kUbList + i] : INFINITY;
                    merge16_groups(ubl);
                }
            }
            if (active && rr == 0 && g == 0 && hasq) {
                // the unit's K smallest kept bounds (K distinct rows) join the query's list; a
                // unit that no longer fits offers its K-th bound instead
                const int base = atomicAdd(&a.ub_cnt[q], a.K);
                uint2* dst = a.ub_list + (size_t)q * a.ub_cap;
                const int row0 = a.vec_off[cid] + vb;
                float uk = INFINITY;
#pragma unroll
                for (int i = 0; i < kUbList; ++i) {
                    if (i < a.K && base + i < a.ub_cap) dst[base + i] = row_entry(ubl[i], row0);
                    if (i == a.K - 1) uk = ubl[i];
                }
                if (base + a.K > a.ub_cap && uk < INFINITY)
                    atomicMin(&a.ub_best[q], __float_as_uint(uk));
            }
        } else {
            if (active) {
                float* s_ub = s_ubl[wid];
#pragma unroll
                for (int i = 0; i < kUbList; ++i) s_ub[j * 64 + g * kUbList + i] = ubl[i];
            }
            __syncthreads();
            if (active && rr == 0) {
                for (int jj = 0; jj < nq; ++jj) {
                    WaveList<64> L;
                    L.init();
                    for (int r2 = 0; r2 < R; ++r2)
                        L.insert(key_of((double)s_ubl[wid + r2][jj * 64 + lane]), lane);
                    // lane i holds the unit's i-th smallest kept bound: the first K join the
                    // query's list
                    const int qq = __shfl(q, jj, kWave);
                    const int nl = ub_per_unit(a.K);
                    int base = 0;
                    if (lane == 0) base = atomicAdd(&a.ub_cnt[qq], nl);
                    base = __shfl(base, 0, kWave);
                    const float uv = L.k0 == kKeyInvalid ? INFINITY : (float)dist_of(L.k0);
                    if (lane < nl && base + lane < a.ub_cap)
                        a.ub_list[(size_t)qq * a.ub_cap + base + lane] =
                            row_entry(uv, a.vec_off[cid] + vb);
                    // K <= 64: the unit's own K-th bound, when its entries did not fit
                    if (a.K <= 64 && lane == a.K - 1 && base + nl > a.ub_cap && uv < INFINITY)
                        atomicMin(&a.ub_best[qq], __float_as_uint(uv));
                }
            }
        }
        if (tid == 0) s_unit[(it + 1) & 1] = nblk > 0 ? nxt : atomicAdd(ctr, 1);
    }
    // telemetry is counted by the lower-bound pass alone, which scans every probed pair once
}

template __global__ void ub_scan_kernel<1, 4>(BatchArgs);
template __global__ void ub_scan_kernel<2, 4>(BatchArgs);
template __global__ void ub_scan_kernel<3, 4>(BatchArgs);
template __global__ void ub_scan_kernel<4, 4>(BatchArgs);
template __global__ void ub_scan_kernel<1, 16>(BatchArgs);
template __global__ void ub_scan_kernel<2, 16>(BatchArgs);
template __global__ void ub_scan_kernel<3, 16>(BatchArgs);
template __global__ void ub_scan_kernel<4, 16>(BatchArgs);
template __global__ void ub_scan_kernel<5, 4>(BatchArgs);
template __global__ void ub_scan_kernel<6, 4>(BatchArgs);
template __global__ void ub_scan_kernel<7, 4>(BatchArgs);
template __global__ void ub_scan_kernel<8, 4>(BatchArgs);
template __global__ void ub_scan_kernel<9, 4>(BatchArgs);
template __global__ void ub_scan_kernel<10, 4>(BatchArgs);
template __global__ void ub_scan_kernel<11, 4>(BatchArgs);
template __global__ void ub_scan_kernel<12, 4>(BatchArgs);
template __global__ void ub_scan_kernel<13, 4>(BatchArgs);
template __global__ void ub_scan_kernel<14, 4>(BatchArgs);
template __global__ void ub_scan_kernel<15, 4>(BatchArgs);
template __global__ void ub_scan_kernel<16, 4>(BatchArgs);
template __global__ void ub_scan_kernel<5, 16>(BatchArgs);
template __global__ void ub_scan_kernel<6, 16>(BatchArgs);
template __global__ void ub_scan_kernel<7, 16>(BatchArgs);
template __global__ void ub_scan_kernel<8, 16>(BatchArgs);
template __global__ void ub_scan_kernel<9, 16>(BatchArgs);
template __global__ void ub_scan_kernel<10, 16>(BatchArgs);
template __global__ void ub_scan_kernel<11, 16>(BatchArgs);
template __global__ void ub_scan_kernel<12, 16>(BatchArgs);
template __global__ void ub_scan_kernel<13, 16>(BatchArgs);
template __global__ void ub_scan_kernel<14, 16>(BatchArgs);
template __global__ void ub_scan_kernel<15, 16>(BatchArgs);
template __global__ void ub_scan_kernel<16, 16>(BatchArgs);

// Seeding threshold, one wave per query.  Its list holds each seeding unit's min(K, 64) smallest
// bounds u with their rows (all distinct rows); the K smallest (u, position) entries are the
// query's seeds:
//   tau_ub = the K-th smallest u (K rows have distance <= it), also over ub_best (a unit's own
//            K-th bound when the list was full), squared and mapped back through the rotation
//            (u^2 / sigma_min^2, margin 1e-6 as the reference's Stage X);
//   tau_x  = the largest canonical float64 distance of the K seeds, each refined here (K distinct
//            rows have distance <= it; never above tau_ub of the same K rows);
//   tau    = min(tau_ub, tau_x).
// The seeds with distance <= tau become the query's first candidates, already refined
// (seed_cnt); the refine of the lower-bound pass skips them.  A query with fewer than K listed
// bounds, or a seed without a recorded row, keeps tau_ub (+inf without bounds) and no seeds.
// A list longer than ub_cap keeps its first ub_cap entries: the K-th smallest of a subset is
// still a bound.
template <int KP, int DQ>
__global__ __launch_bounds__(256) void ub_kth_kernel(BatchArgs a) {
    __shared__ double s_q64[kWavesPerBlock][DQ];
    __shared__ float s_stage[kWavesPerBlock][kStageCh][kWave + 1];
    __shared__ int32_t s_pos[kWavesPerBlock][KP];
    const int lane = threadIdx.x & 63, wid = (int)(threadIdx.x >> 6);
    const int q = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + wid);
    if (q >= a.B) return;
    const int K = a.K, n = min(a.ub_cnt[q], a.ub_cap);
    const float ubest = __uint_as_float(a.ub_best[q]);
    double tau = ubest < INFINITY ? (double)ubest * ubest / a.rot_sq_min * (1.0 + 1e-6) : INFINITY;
    if (n >= K) {
        const uint2* lst = a.ub_list + (size_t)q * a.ub_cap;
        WaveList<KP> L;
        L.init();
        for (int i0 = 0; i0 < n; i0 += kWave) {
            const int i = i0 + lane;
            const uint2 e = i < n ? lst[i] : make_uint2(0u, 0u);
            L.insert(i < n ? key_of((double)__uint_as_float(e.x)) : kKeyInvalid,
                     i < n ? (int32_t)e.y : kIdInvalid);
        }
        uint64_t kk;
        int32_t ki;
        L.at(K - 1, kk, ki);
        const double u = kk != kKeyInvalid ? dist_of(kk) : INFINITY;
        if (u < (double)INFINITY) tau = fmin(tau, u * u / a.rot_sq_min * (1.0 + 1e-6));
        // exact seeding: every one of the K smallest entries is finite and has its row
        bool ok = lane >= K || (L.k0 != kKeyInvalid && L.i0 >= 0);
        if constexpr (KP > 64) ok = ok && (lane + kWave >= K || (L.k1 != kKeyInvalid && L.i1 >= 0));
        if (u < (double)INFINITY && __ballot(!ok) == 0ull && a.fine_mode) {
            // fine codes: the K seeds' upper bounds from HBM; no row crosses PCIe here and
            // no seed is listed (the lower-bound pass lists every row with d64 <= tau)
            for (int d = lane; d < a.D_pad; d += kWave) s_q64[wid][d] = a.xrot64[(size_t)q * a.D_pad + d];
            wave_sync();
            const double qe = sqrt(a.qep[q]) * (1.0 + 1e-12);
            double mx = 0.0;
            for_chunks<KP>([&](auto cc) __attribute__((always_inline)) {
                constexpr int h = decltype(cc)::value;
                uint64_t hk;
                int32_t pos;
                list_chunk<h>(L, hk, pos);
                if (h * kWave + lane < K) {
                    double lb, ub;
                    fine_row_bounds(a, s_q64[wid], qe, pos, lb, ub);
                    mx = fmax(mx, ub);
                }
            });
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) mx = fmax(mx, shfl_f64(mx, lane ^ o));
            tau = fmin(tau, mx);
        } else if (u < (double)INFINITY && __ballot(!ok) == 0ull) {
            if (lane < K) s_pos[wid][lane] = L.i0;
            if constexpr (KP > 64)
                if (lane + kWave < K) s_pos[wid][kWave + lane] = L.i1;
            for (int d = lane; d < a.D; d += kWave) s_q64[wid][d] = (double)a.xq[(size_t)q * a.D + d];
            wave_sync();
            double dv[KP / kWave];
            double mx = 0.0;
#pragma unroll
            for (int h = 0; h < KP / kWave; ++h) {
                const int nr = min(kWave, K - h * kWave);
                dv[h] = 0.0;
                if (nr > 0) {
                    dv[h] = refine_rows(a.xb, a.xb8, a.D, s_pos[wid] + h * kWave, nr, s_stage[wid],
                                            s_q64[wid]);
                    if (lane < nr) mx = fmax(mx, dv[h]);
                }
            }
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) mx = fmax(mx, shfl_f64(mx, lane ^ o));
            tau = fmin(tau, mx);
            if (a.host_rows && a.xb_host && lane == 0) atomicAdd(a.host_rows, (unsigned long long)K);
            // the seeds as the first candidates (refined): those within tau
            int cnt = 0;
            uint64_t* ck = a.cand_key + (size_t)q * a.cap;
            int32_t* ci = a.cand_id + (size_t)q * a.cap;
#pragma unroll
            for (int h = 0; h < KP / kWave; ++h) {
                const int r = h * kWave + lane;
                const bool keep = r < K && dv[h] <= tau;
                const uint64_t m = __ballot(keep);
                if (keep) {
                    const int slot = cnt + mask_rank(m);
                    ck[slot] = key_of(dv[h]);
                    ci[slot] = a.orig_ids[s_pos[wid][r]];
                }
                cnt += __popcll(m);
            }
            if (lane == 0) {
                a.cand_cnt[q] = cnt;
                a.seed_cnt[q] = cnt;
                if (a.stats && cnt) atomicAdd(&a.stats[(q % kStatSlots) * 4 + 3], (unsigned long long)cnt);
            }
        }
    }
    if (lane == 0) a.tau[q] = tau;
}

template __global__ void ub_kth_kernel<64, 256>(BatchArgs);
template __global__ void ub_kth_kernel<64, 1024>(BatchArgs);
template __global__ void ub_kth_kernel<128, 256>(BatchArgs);
template __global__ void ub_kth_kernel<128, 1024>(BatchArgs);

// ---------------------------------------------------------------------------------------------
// Lower-bound pass.
//
// lb_prep_kernel: one 32-lane group per weight group, one lane per pair, after the seeding pass.
// For pair (q, c) with t_q = sqrt(tau_q * rot_sq_max) (1 + 1e-12) + e_q the lower-bound
// condition is (norm form against sqrt(tau) scaled to the rotated space)
//     A - r^2 - 2 t_q r  <=  c1 (acc + cW) + G,   G = 2 err - Q + t_q^2,  c1 = 2 s,
// with acc = sum (c - 128) w_int (exact int32).  Two forms of it are prepared:
//   float:   fma(c2f, r, P) <= fma(c1f, float(acc), H32), P = A_lo - r^2 in float32,
//            c2f <= -2 t_q, H32 >= c1 cW + G + slack; each of the 4 f32 roundings is at most
//            2^-24 of a term bounded by X = A_max + r_max^2 + 2 t_q r_max + c1 acc_max + |H|
//            (A_max = 255^2 sum delta^2, r_max = 2 sqrt(sum eps^2), acc_max = 128 sum |w_int|),
//            so slack = 2^-22 X covers them all;
//   integer: acc + kq >= thr_x with thr_x <= (A_lo - r (r + 2 t_w)) / c1 per vector (t_w the
//            group's largest t_q) and kq >= cW + G / c1 - 2 (t_w - t_q) r_lo / c1 (r_lo <= r_x
//            over the cluster): A - r^2 - 2 t_q r >= A - r (r + 2 t_w) + 2 (t_w - t_q) r_lo.
//            G / c1 is exact (c1 is a power of two); mg covers the roundings of G and of the
//            sums.  The group takes it iff every query has a threshold, all share c1 and
//            |kq| <= 2^30 (pair_prep_kernel keeps |acc| < 2^30, so the int32 sum cannot
//            overflow).
__global__ __launch_bounds__(256) void lb_prep_kernel(BatchArgs a) {
    static_assert(kGroupQ == 32, "one 32-lane half wave per weight group");
    const int tid = threadIdx.x, lane = tid & 63, slot = tid & 31;
    const int gi = blockIdx.x * (kBlock / kGroupQ) + (tid >> 5);
    if (a.tau_sq_out)  // the seeded thresholds, rounded up to float32, for the caller
        for (int q = blockIdx.x * kBlock + tid; q < a.B; q += gridDim.x * kBlock)
            a.tau_sq_out[q] = __double2float_ru(a.tau[q]);
    if (gi >= min(a.grp_off[a.nlist], a.max_groups)) return;  // whole 32-lane groups
    const int2 grp = a.groups[gi];
    const bool valid = slot < grp.y;
    const int p = grp.x + (valid ? slot : 0);
    const int q = a.pair_qid[p], c = a.pair_cid[p];
    const PairRec pr = a.prec[p];
    const double Qp = pr.Qp, err_q = pr.err_q, cW = pr.cW, c1 = pr.c1;
    const double tq = sqrt(a.tau[q] * a.rot_sq_max) * (1.0 + 1e-12) + pr.e_q;
    const bool thr = tq < 1e30;
    LbRec L;
    L.kq = 0;
    L.c1f = 0.0f;
    L.c2f = 0.0f;
    L.H32 = INFINITY;  // no threshold: every row passes
    double Kd = 0.0, mg = 0.0;
    float tqf = 0.0f;
    if (thr) {
        const double G = 2.0 * err_q - Qp * (1.0 - a.sum_rel) + tq * tq;
        const double H = c1 * cW + G;
        const double X = pr.a_max + pr.r_max * pr.r_max + 2.0 * tq * pr.r_max + c1 * pr.acc_max +
                         fabs(H);
        const double slack = 0x1p-22 * X * (1.0 + 1e-6) + 1e-30;
        L.H32 = __double2float_ru(H + slack);
        L.c1f = (float)c1;
        L.c2f = -__double2float_ru(2.0 * tq);
        Kd = cW + G / c1;
        mg = 0x1p-50 * (fabs(Kd) + (2.0 * err_q + Qp + tq * tq) / c1);
        tqf = __double2float_ru(tq);
    }
    // group reductions over the 32 lanes of this weight group
    const double c1_0 = shfl_f64(c1, lane & ~31);
    int bad = valid && (!thr || c1 != c1_0);
    float tqw = valid ? tqf : 0.0f;
    // lo_l2 / 256 is exact in float64 (a power of two), rounded up to float32
    float low = valid && a.vec_cn ? __double2float_ru(pr.lo_l2 * 0x1p-8) : 0.0f;
#pragma unroll
    for (int o = 1; o < kGroupQ; o <<= 1) {
        bad |= __shfl_xor(bad, o, kWave);
        tqw = fmaxf(tqw, __shfl_xor(tqw, o, kWave));
        low = fmaxf(low, __shfl_xor(low, o, kWave));
    }
    bool ok = !bad && c1_0 >= 0x1p-100 && c1_0 <= 0x1p100;
    if (ok && valid) {
        const double r_lo = a.cbound[kCbStride * c + 2];
        const double corr = 2.0 * ((double)tqw - tq) * r_lo / c1_0 * (1.0 - 0x1p-50);
        const double kd = ceil(Kd - corr + (mg + 0x1p-50 * fabs(corr)));
        if (fabs(kd) <= 0x1p30) L.kq = (int)kd;
        else ok = false;
    }
    int nok = valid && !ok;
#pragma unroll
    for (int o = 1; o < kGroupQ; o <<= 1) nok |= __shfl_xor(nok, o, kWave);
    L.int_ok = !nok;
    L.tqw = tqw;
    L.inv_c1w = L.int_ok ? (float)(1.0 / c1_0) : 0.0f;  // a power of two in [2^-100, 2^100]
    // The hi-plane prefilter's allowance for the lo plane: with row norms, lo_w * 256 * cn_x per
    // row (Cauchy-Schwarz against the group's largest lo-plane norm), else lo_max per query
    // (|kq| <= 2^30 and lo_max <= 2^24: no int32 overflow).
    L.lo_w = low;
    L.kq_pre = !L.int_ok ? 0 : a.vec_cn ? L.kq : L.kq + (int)pr.lo_max;
    if (valid) {
        a.lbr[p] = L;
        a.lbk[p] = make_int2(L.kq, L.kq_pre);
    }
}


// Pass B, narrow layout (D_pad <= 256; LDS blocks of 128 rows up to D_pad 128, else 64), every
// probe of a unit's cluster slice.  Queries are the rows of the matrix-core product (A operand, 16 per MFMA, weights held
// in registers) and vectors its columns (B operand, read from LDS), so a lane's four results
// (rows 4 g + r, column j = lane & 15) share one vector and the integer test needs one int32
// threshold per lane: max over the lane's rows of S = acc + kq against thr_x.  Each wave owns
// 32 queries (two 16-row halves: eight MFMAs per 64-dim code fragment pair read from LDS), a
// unit up to 128, so a slice's codes are staged once per 128 queries of the cluster.  Block
// b + 1's code cells and row scalars (A_lo, r) move global -> LDS directly (no staging
// registers) while the waves scan block b; each wave turns the row scalars into its own int32
// thresholds once per block.  Survivors are queued per wave in LDS and appended with one atomic
// per query and flush.
template <int KS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KS <= 2 ? 4 : 1)))
void lb_scan_kernel(BatchArgs a) {
    static_assert(KS <= 4, "narrow layout: D_pad <= 256");
    constexpr int BV = 64;               // rows of one cell run (G16 * 64 cells)
    constexpr int SB = KS <= 2 ? 2 : 1;  // cell runs per LDS block
    constexpr int BR = SB * BV;          // rows per LDS block
    constexpr int QW = 32;               // queries per wave
    // Two LDS blocks: one is scanned while the next one's loads are in flight.  A block is as
    // large as 32 KB of codes allows, so that its fixed costs (the barrier, the wave's
    // thresholds, the load issue) are spread over as many tiles as possible.
    constexpr int NBUF = 2;
    __shared__ uint4 s_codes[NBUF][SB][KS * 4 * BV];
    __shared__ __align__(16) float s_A[NBUF][BR];
    __shared__ __align__(16) float s_r[NBUF][BR];
    __shared__ __align__(16) float s_cn[NBUF][BR];  // row code norms (vec_cn)
    __shared__ uint32_t s_sq[kWavesPerBlock][kLbQ];
    __shared__ int s_scnt[kWavesPerBlock][QW], s_sbase[kWavesPerBlock][QW];
    __shared__ float4 s_qf[kWavesPerBlock][QW];  // per query slot: (c1f, c2f, H32, -)
    // per query slot: kq, the lo-plane accumulators' start (empty slots INT_MIN); read only by
    // tiles that pass the hi-plane prefilter, so it is not held in registers
    __shared__ __align__(16) int s_kq[kWavesPerBlock][QW];
    __shared__ int s_unit[2];
    __shared__ int4 s_urec[2];  // the units' records, fetched during the previous unit

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int u0 = a.unit_off[a.unit_beg], u1 = min(a.unit_off[a.unit_end], a.max_units);
    const int nx = (max(u1 - u0, 0) + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int rb = u0 + xcd * nx, re = min(u1, rb + nx);
    int32_t* ctr = a.ctr + xcd * kCtrStride;
    const int T = a.T, G16 = a.D_pad >> 4;
    unsigned long long st_cand = 0, st_surv = 0;
    if (lane < QW) s_scnt[wid][lane] = 0;

    // Next unit: its counter value is taken three blocks before the current unit ends and its
    // record moves global -> LDS two blocks before (thread 0, a direct load into s_urec), both
    // published at the end of the unit (slot (it + 1) & 1, read at the start of unit it + 1;
    // its previous read, at the start of unit it - 1, is separated from the writes by the
    // barrier at the top of unit it).  The explicit waits keep the LDS write and the direct
    // load ahead of the barrier.
    if (tid == 0) {
        const int u = atomicAdd(ctr, 1);
        s_unit[0] = u;
        if (rb + u < re) s_urec[0] = a.units[rb + u];
    }
    for (int it = 0;; ++it) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + rb;
        if (ui < rb || ui >= re) break;
        int nxt = 0;
        const int4 un = s_urec[it & 1];
        const int cid = __builtin_amdgcn_readfirstlane(un.x & 0xfffff),
                  cnt = __builtin_amdgcn_readfirstlane(un.x >> 20),
                  start = __builtin_amdgcn_readfirstlane(un.y),
                  vb = __builtin_amdgcn_readfirstlane(un.z), ve = __builtin_amdgcn_readfirstlane(un.w);
        const int G = (cnt + QW - 1) / QW;  // 32-query blocks (1..4)
        const int R = kWavesPerBlock / G;   // waves sharing a block split its tiles
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(QW, cnt - gq * QW) : 0;
        const bool two = nq > 16;           // the second half holds queries (wave-uniform)
        const int v0 = a.vec_off[cid];
        const int t0 = a.tile_off[cid];
        const int pb = start + gq * QW;     // the wave's first pair: a weight group's first

        // ---- this wave's queries: weight rows and the constants of lb_prep_kernel ----
        v4i whi[2][KS], wlo[2][KS], hq4[2];
        bool int_ok = false;
        float tqw = 0.0f, inv_c1w = 0.0f, lo_w = 0.0f;
        if (active) {
            // every prologue load is issued before the first use (one memory round trip): the
            // group's constants, the (kq, kq_pre) of the lane's rows (lbk is padded by 32
            // entries, so rows past the unit stay inside it), the weight rows
            const LbRec L0 = a.lbr[pb];
            int2 kk[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) kk[h][r] = a.lbk[pb + 16 * h + 4 * g + r];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int qi = 16 * h + j;  // the A row this lane supplies
                const bool hv = qi < nq;
                const int8_t* hp = a.pw + (size_t)(pb + (hv ? qi : 0)) * 2 * a.DP + g * 16;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const v4i vh = *reinterpret_cast<const v4i*>(hp + ks * 64);
                    const v4i vl = *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64);
                    whi[h][ks] = hv ? vh : v4i{0, 0, 0, 0};
                    wlo[h][ks] = hv ? vl : v4i{0, 0, 0, 0};
                }
            }
            int_ok = __builtin_amdgcn_readfirstlane(L0.int_ok) != 0;
            tqw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L0.tqw)));
            inv_c1w = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L0.inv_c1w)));
            lo_w = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L0.lo_w)));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // C rows this lane receives: queries 16 h + 4 g + r (empty rows: INT_MIN)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int qr = 16 * h + 4 * g + r;
                    // hi-plane start: ceil(kq_pre / 256) (|kq_pre| < 2^31 - 255); empty rows
                    // start far below any threshold
                    hq4[h][r] = qr < nq && int_ok ? (kk[h][r].y + 255) >> 8 : -(1 << 25);
                }
            }
            if (lane < QW) {
                const bool hv = lane < nq;
                const LbRec L = a.lbr[pb + (hv ? lane : 0)];
                // integer groups: kq - 256 ceil(kq_pre / 256), the lo plane's start after the
                // row's hi-plane sum (which began at ceil(kq_pre / 256)) is shifted left by 8
                // (mod 2^32: the true sum 256 acc_hi + kq fits in int32)
                s_kq[wid][lane] = !hv ? INT_MIN
                                : int_ok ? (int)((uint32_t)L.kq - ((uint32_t)((L.kq_pre + 255) >> 8) << 8))
                                         : L.kq;
                // .w: the slot's query id, for the survivor flush (no global reads there)
                s_qf[wid][lane] = hv ? make_float4(L.c1f, L.c2f, L.H32, __int_as_float(a.pair_qid[pb + lane]))
                                     : make_float4(0.0f, 0.0f, -INFINITY, 0.0f);  // never passes
            }
        }
        // residual-norm band: lane l < nq holds query slot l's |q - c| and threshold
        float l1_dqc = 0.0f;
        double l1_tau = -1.0;  // lanes without a query skip every tile
        if (a.use_l1 && active && lane < nq) {
            l1_dqc = a.pair_dqc[pb + lane];
            l1_tau = a.tau[a.pair_qid[pb + lane]];
        }

        // ---- survivor queue (entries li << 5 | query slot) ----
        int nsq = 0;
        // the integer thresholds th of the block's rows sb * 64 + lane, and their hi-plane form
        // thh = floor((th - 1) / 256) + 1 - cb (256 (h + cb) < th iff h < thh)
        int thr_r[SB], thh_r[SB];
        auto flush = [&]() __attribute__((always_inline)) {
            for (int e = lane; e < nsq; e += kWave) atomicAdd(&s_scnt[wid][s_sq[wid][e] & 31u], 1);
            __builtin_amdgcn_wave_barrier();
            if (lane < QW) {
                const int c = s_scnt[wid][lane];
                s_sbase[wid][lane] = c ? atomicAdd(&a.cand_cnt[__float_as_int(s_qf[wid][lane].w)], c) : 0;
                s_scnt[wid][lane] = 0;
            }
            __builtin_amdgcn_wave_barrier();
            for (int e = lane; e < nsq; e += kWave) {
                const uint32_t ent = s_sq[wid][e];
                const int jj = (int)(ent & 31u);
                const int slot = s_sbase[wid][jj] + atomicAdd(&s_scnt[wid][jj], 1);
                if (slot < a.cap)
                    a.cand_id[(size_t)__float_as_int(s_qf[wid][jj].w) * a.cap + slot] = v0 + (int)(ent >> 5);
            }
            __builtin_amdgcn_wave_barrier();
            if (lane < QW) s_scnt[wid][lane] = 0;
            if (a.stats) st_surv += (unsigned long long)nsq;
            nsq = 0;
        };

        // ---- rare: queue the passing (query row, vector) entries of a tile; `pass(h, r)` is
        // this lane's test of row 4 g + r of half h against its vector li ----
        auto queue = [&](auto pass, bool has2, int li) __attribute__((always_inline)) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (h == 1 && !has2) break;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool ps = pass(h, r);
                    const uint64_t pm = __ballot(ps);
                    if (__builtin_expect(pm == 0ull, 1)) continue;
                    if (__builtin_expect(nsq + __popcll(pm) > kLbQ, 0)) flush();
                    if (ps) {
                        const int idx = __builtin_amdgcn_mbcnt_hi(
                            (uint32_t)(pm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)pm, 0u));
                        s_sq[wid][nsq + idx] = ((uint32_t)li << 5) | (uint32_t)(16 * h + 4 * g + r);
                    }
                    nsq += __popcll(pm);
                }
            }
        };

        // ---- one 16-vector tile: load_b reads its code fragments (the B operands) from LDS,
        // tile_b runs it on them; INT = the integer test, TWO = both halves hold queries ----
        auto load_b = [&](int buf, int t, v4i (&Bo)[KS]) __attribute__((always_inline)) {
            const uint4* blk = s_codes[buf][t >> 2];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 v = blk[(ks * 4 + g) * BV + (t & 3) * 16 + j];
                Bo[ks] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
        };
        auto tile_b = [&](auto int_c, auto two_c, int buf, int t, int li0, const v4i (&B)[KS]) __attribute__((always_inline)) {
            constexpr bool INT = decltype(int_c)::value, TWO = decltype(two_c)::value;
            // the thresholds of column j (row t * 16 + j of the block) are held by lane
            // (t & 3) * 16 + j in its run's registers
            const int src = (((t & 3) << 4) | j) << 2;
            int thh = 0;
            if constexpr (INT)
                thh = __builtin_amdgcn_ds_bpermute(src, SB == 1 || (t >> 2) == 0 ? thh_r[0] : thh_r[SB - 1]);
            v4i h0 = {0, 0, 0, 0}, l0 = {0, 0, 0, 0}, h1 = {0, 0, 0, 0}, l1 = {0, 0, 0, 0};
            if constexpr (INT) {
                // Hi plane first, started at ceil(kq_pre / 256) per row, so that
                // S = 256 acc_hi + acc_lo + kq <= 256 h + 256 cb_x with cb_x the row's lo-plane
                // allowance (0 when kq_pre carries lo_max, else ceil(cn_x lo_w) >= |acc_lo| / 256
                // by Cauchy-Schwarz).  A tile whose rows all have h < thh (256 (h + cb_x) < th)
                // fails the exact test too and costs no lo-plane work.
                h0 = hq4[0];
                h1 = hq4[1];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    h0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi[0][ks], B[ks], h0, 0, 0, 0);
                    if constexpr (TWO)
                        h1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi[1][ks], B[ks], h1, 0, 0, 0);
                }
                int mh = max(max(h0[0], h0[1]), max(h0[2], h0[3]));
                if constexpr (TWO) mh = max(mh, max(max(h1[0], h1[1]), max(h1[2], h1[3])));
                if (__builtin_expect(__ballot(mh >= thh) == 0ull, 1)) return;
                // the lo plane continues from 256 (plain hi sum) + kq in the same registers
                {
                    // the LDS address formed here (hoisted, it would stay live for the unit)
                    int gl = g;
                    asm volatile("" : "+v"(gl));
                    const v4i k0 = *reinterpret_cast<const v4i*>(&s_kq[wid][4 * gl]);
                    v4i k1 = {0, 0, 0, 0};
                    if constexpr (TWO) k1 = *reinterpret_cast<const v4i*>(&s_kq[wid][16 + 4 * gl]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        h0[r] = (int)(((uint32_t)h0[r] << 8) + (uint32_t)k0[r]);
                        if constexpr (TWO) h1[r] = (int)(((uint32_t)h1[r] << 8) + (uint32_t)k1[r]);
                    }
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    h0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo[0][ks], B[ks], h0, 0, 0, 0);
                    if constexpr (TWO)
                        h1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo[1][ks], B[ks], h1, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    h0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi[0][ks], B[ks], h0, 0, 0, 0);
                    l0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo[0][ks], B[ks], l0, 0, 0, 0);
                    if constexpr (TWO) {
                        h1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(whi[1][ks], B[ks], h1, 0, 0, 0);
                        l1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wlo[1][ks], B[ks], l1, 0, 0, 0);
                    }
                }
            }
            // rows 4 g + r (queries), column j (vector li0 + j): S = acc + kq, exact in int32
            int S[2][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                S[0][r] = INT ? h0[r] : (h0[r] << 8) + l0[r];
                S[1][r] = TWO ? (INT ? h1[r] : (h1[r] << 8) + l1[r]) : INT_MIN;
            }
            const int li = li0 + j;
            if constexpr (INT) {
                const int th =
                    __builtin_amdgcn_ds_bpermute(src, SB == 1 || (t >> 2) == 0 ? thr_r[0] : thr_r[SB - 1]);
                int m = max(max(S[0][0], S[0][1]), max(S[0][2], S[0][3]));
                if constexpr (TWO) m = max(m, max(max(S[1][0], S[1][1]), max(S[1][2], S[1][3])));
                if (__builtin_expect(__ballot(m >= th) == 0ull, 1)) return;
                queue([&](int h, int r) __attribute__((always_inline)) { return S[h][r] >= th; }, TWO, li);
            } else {
                const float Av = s_A[buf][t * 16 + j], rv = s_r[buf][t * 16 + j];
                const float P = fmaf(-rv, rv, Av);
                const bool in = li < ve;
                auto pass = [&](int h, int r) __attribute__((always_inline)) {
                    const float4 c = s_qf[wid][16 * h + 4 * g + r];
                    return in && fmaf(c.y, rv, P) <= fmaf(c.x, (float)S[h][r], c.z);
                };
                bool any = false;
#pragma unroll
                for (int h = 0; h < (TWO ? 2 : 1); ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) any |= pass(h, r);
                if (__builtin_expect(__ballot(any) == 0ull, 1)) return;
                queue(pass, TWO, li);
            }
        };
        auto tiles = [&](auto int_c, auto two_c, int buf, int blk0) __attribute__((always_inline)) {
            if (R == 1 && blk0 + BR <= ve) {  // the common case: straight-line tiles, the next
                                              // tile's codes read before this one's branches
                v4i Bc[KS], Bn[KS];
                load_b(buf, 0, Bn);
#pragma unroll
                for (int t = 0; t < BR / 16; ++t) {
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) Bc[ks] = Bn[ks];
                    if (t + 1 < BR / 16) load_b(buf, t + 1, Bn);
                    tile_b(int_c, two_c, buf, t, blk0 + t * 16, Bc);
                }
            } else {
                for (int t = rr; t < BR / 16; t += R) {
                    if (blk0 + t * 16 >= ve) break;
                    v4i Bc[KS];
                    load_b(buf, t, Bc);
                    tile_b(int_c, two_c, buf, t, blk0 + t * 16, Bc);
                }
            }
        };

        // ---- stream the slice through LDS in blocks of SB cell runs ----
        // Block-major cells ([tiles, T / 64, G16, 64]): a cluster's 64-vector runs are
        // consecutive runs of G16 * 64 cells, so rows v0 .. v0 + 63 of the cluster start at
        // cell G16 * v0 and the next block to load is one pointer step away (no per-block
        // tile / slot arithmetic in the scalar unit).
        const uint4* next_blk = a.cells + (size_t)t0 * G16 * T + (size_t)G16 * vb;
        // row norms: without vec_cn the A values stand in (finite; lo_w = 0 then)
        const void* cn_base = a.vec_cn ? (const void*)(a.vec_cn + v0) : (const void*)(a.vec_Ar + v0);
        const int cn_sh = a.vec_cn ? 2 : 3;
        auto gload = [&](int buf, int blk0) __attribute__((always_inline)) {
#pragma unroll
            for (int sb = 0; sb < SB; ++sb) {
                // a run past the slice end loads the block's first run again (its rows are never
                // scanned): the cells after a cluster's last run belong to the next cluster or lie
                // past the array, and every block issues the same loads (the waits count them)
                const uint4* base =
                    (sb == 0 || blk0 + sb * BV < ve ? next_blk + (size_t)sb * G16 * BV : next_blk) +
                    wid * BV;
#pragma unroll
                for (int jj = 0; jj < KS; ++jj)
                    if (wid + 4 * jj < G16)
                        load_lds16(base + (size_t)(4 * jj) * BV, 16u * lane,
                                   &s_codes[buf][sb][(wid + 4 * jj) * BV]);
            }
            if (wid == 0) {  // rows past the slice read the slice's last row (never used)
#pragma unroll
                for (int sb = 0; sb < SB; ++sb) {
                    const uint32_t row = (uint32_t)min(blk0 + sb * BV + lane, ve - 1);
                    load_lds4(a.vec_Ar + v0, 8u * row, &s_A[buf][sb * BV]);
                    load_lds4(a.vec_Ar + v0, 8u * row + 4u, &s_r[buf][sb * BV]);
                    load_lds4(cn_base, row << cn_sh, &s_cn[buf][sb * BV]);
                }
            }
            next_blk += (size_t)G16 * BR;
        };
        const int nblk = (ve - vb + BR - 1) / BR;
        // direct loads this wave issues per block (its code groups, plus the row scalars)
        int nl = wid == 0 ? 3 * SB : 0;
#pragma unroll
        for (int jj = 0; jj < KS; ++jj) nl += wid + 4 * jj < G16 ? SB : 0;
#pragma unroll
        for (int pb0 = 0; pb0 < NBUF - 1; ++pb0)
            if (pb0 < nblk) gload(pb0, vb + pb0 * BR);
        for (int b = 0; b < nblk; ++b) {
            const int buf = b % NBUF;
            // this wave's direct loads of block b have landed: vector memory operations complete
            // in issue order, and only the loads of blocks b + 1 .. b + NBUF - 2 (plus any
            // stores or atomics, which only make the wait longer) were issued after them; the
            // barrier covers everyone's.  It also retires block b - 1, whose buffer is refilled
            // next.
            wait_vmcnt(nl * min(NBUF - 2, nblk - 1 - b));
            __syncthreads();
            if (tid == 0 && b == max(nblk - 3, 0)) nxt = atomicAdd(ctr, 1);
            if (tid == 0 && b == max(nblk - 2, 0) && rb + nxt < re)  // one direct 16-byte load
                load_lds16(a.units + rb, 16u * (uint32_t)nxt, &s_urec[(it + 1) & 1]);
            const int blk0 = vb + b * BR;
            if (b + NBUF - 1 < nblk) gload((b + NBUF - 1) % NBUF, blk0 + (NBUF - 1) * BR);
            if (!active) continue;
            if (a.use_l1) {  // the wave leaves the block when none of its queries reaches its tiles
                const int ta = blk0 / T, tb = (min(blk0 + BR, ve) - 1) / T;
                const float* rm = a.tile_rmm + 2 * (size_t)(t0 + ta);
                bool need = l1_tau >= 0.0 && !l1_skips(l1_dqc, l1_tau, rm[0], rm[1]);
                if (tb != ta) need = need || (l1_tau >= 0.0 && !l1_skips(l1_dqc, l1_tau, rm[2], rm[3]));
                if (__ballot(need) == 0ull) continue;
            }
            if (int_ok) {
#pragma unroll
                for (int sb = 0; sb < SB; ++sb) {
                    const int i = sb * BV + lane;
                    const float A = s_A[buf][i], r = s_r[buf][i];
                    const int th = lb_thr(A, r, tqw, inv_c1w);  // rows past the slice: INT_MAX
                    thr_r[sb] = blk0 + i < ve ? th : INT_MAX;
                    // the lo plane's allowance in hi units: ceil(cn lo_w) >= |acc_lo| / 256
                    // (the product's rounding is covered by the 2^-20 raise)
                    const float p = s_cn[buf][i] * lo_w;
                    thh_r[sb] = ((thr_r[sb] - 1) >> 8) + 1 - (int)ceilf(fmaf(p, 0x1p-20f, p));
                }
                if (two) tiles(std::true_type{}, std::true_type{}, buf, blk0);
                else tiles(std::true_type{}, std::false_type{}, buf, blk0);
            } else {
                if (two) tiles(std::false_type{}, std::true_type{}, buf, blk0);
                else tiles(std::false_type{}, std::false_type{}, buf, blk0);
            }
        }
        if (a.stats && active && rr == 0)
            st_cand += (unsigned long long)nq * (unsigned long long)(ve - vb);
        if (nsq > 0) flush();
        if (tid == 0) {
            if (nblk == 0) {  // (slices are never empty; kept for safety)
                nxt = atomicAdd(ctr, 1);
                if (rb + nxt < re) s_urec[(it + 1) & 1] = a.units[rb + nxt];
            }
            s_unit[(it + 1) & 1] = nxt;
        }
    }

    if (a.stats && lane == 0) {
        const int slot = (int)(blockIdx.x % kStatSlots) * 4;
        atomicAdd(&a.stats[slot + 0], st_cand);
        atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)(a.D_pad));
        atomicAdd(&a.stats[slot + 2], st_surv);
    }
}

template __global__ void lb_scan_kernel<1>(BatchArgs);
template __global__ void lb_scan_kernel<2>(BatchArgs);
template __global__ void lb_scan_kernel<3>(BatchArgs);
template __global__ void lb_scan_kernel<4>(BatchArgs);

// Pass B, wide layout (256 < D_pad <= 1024, one 16-vector tile per LDS block in a ring):
// units of <= 64 queries, each wave owns 16 (the MFMA's B columns; vectors are its A rows)
// or, when a unit holds fewer, several waves share 16 queries and split each block's 64-dim
// steps (replicas, partial sums exchanged through LDS).  Block loads, thresholds and the
// survivor queue as in lb_scan_kernel.
template <int KS>
__global__ __launch_bounds__(256) void lb_scan_wide_kernel(BatchArgs a) {
    constexpr int BV = block_vectors(KS);
    static_assert(BV == 16, "wide layout");
    // code buffers, row scalars and replica partial sums as in ub_scan_kernel
    constexpr int NBC = kWideAhead + 1;
    __shared__ uint4 s_codes[NBC][KS * 4 * BV];
    constexpr int NAB = 8, NP = 2;
    __shared__ __align__(16) float s_A[NAB][BV];
    __shared__ __align__(16) float s_r[NAB][BV];
    __shared__ int4 s_part[NP][NP > 1 ? kWavesPerBlock : 1][NP > 1 ? kWave : 1];
    __shared__ __align__(16) int s_thr[2][kWavesPerBlock][BV];
    __shared__ uint32_t s_sq[kWavesPerBlock][kLbQ];
    __shared__ int s_scnt[kWavesPerBlock][kWaveQ], s_sbase[kWavesPerBlock][kWaveQ],
        s_sqid[kWavesPerBlock][kWaveQ];
    __shared__ float4 s_qf[kWavesPerBlock][kWaveQ];  // per query slot: (c1f, c2f, H32, -)
    __shared__ int s_unit[2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int u0 = a.unit_off[a.unit_beg], u1 = min(a.unit_off[a.unit_end], a.max_units);
    const int nx = (max(u1 - u0, 0) + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int rb = u0 + xcd * nx, re = min(u1, rb + nx);
    int32_t* ctr = a.ctr + xcd * kCtrStride;
    const int T = a.T, G16 = a.D_pad >> 4;
    unsigned long long st_cand = 0, st_surv = 0;
    if (lane < kWaveQ) s_scnt[wid][lane] = 0;

    // Next unit's counter value: taken two blocks before the current unit ends, published in
    // s_unit at its end (slot (it + 1) & 1, read at the start of unit it + 1; its previous read,
    // at the start of unit it - 1, is separated from the write by the barrier at the top of
    // unit it).  The explicit LDS wait keeps that write ahead of the barrier.
    if (tid == 0) s_unit[0] = atomicAdd(ctr, 1);
    for (int it = 0;; ++it) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + rb;
        if (ui < rb || ui >= re) break;
        int nxt = 0;
        const int4 un = a.units[ui];
        const int cid = un.x & 0xfffff, cnt = un.x >> 20, start = un.y, vb = un.z, ve = un.w;
        const int G = (cnt + kWaveQ - 1) / kWaveQ;
        const int R = kWavesPerBlock / G;
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(kWaveQ, cnt - gq * kWaveQ) : 0;
        const bool hasq = j < nq;
        const int v0 = a.vec_off[cid];
        const int t0 = a.tile_off[cid];

        // ---- this wave's queries: weight planes and the constants of lb_prep_kernel ----
        v4i bhi[KS], blo[KS];
        int q = 0, kq = 0;
        float4 qf = make_float4(0.0f, 0.0f, -INFINITY, 0.0f);  // no query: nothing passes
        bool int_ok = false;
        float tqw = 0.0f, inv_c1w = 0.0f;
        if (active) {
            const int pj = start + gq * kWaveQ + (hasq ? j : 0);
            q = a.pair_qid[pj];
            const int8_t* hp = a.pw + (size_t)pj * 2 * a.DP + g * 16;
            if (R == 1) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    bhi[ks] = *reinterpret_cast<const v4i*>(hp + ks * 64);
                    blo[ks] = *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64);
                }
            } else {
                // wide layout with R replicas: slot i holds step rr + i R (zero past KS)
#pragma unroll
                for (int i = 0; i < KS; ++i) {
                    const int ks = rr + i * R;
                    bhi[i] = ks < KS ? *reinterpret_cast<const v4i*>(hp + ks * 64) : v4i{0, 0, 0, 0};
                    blo[i] = ks < KS ? *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64)
                                     : v4i{0, 0, 0, 0};
                }
            }
            const LbRec L = a.lbr[pj];
            int_ok = __builtin_amdgcn_readfirstlane(L.int_ok) != 0;  // lane 0 has a query
            tqw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L.tqw)));
            inv_c1w = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(L.inv_c1w)));
            if (hasq) {
                kq = int_ok ? L.kq : 0;
                qf = make_float4(L.c1f, L.c2f, L.H32, 0.0f);
            } else {
                kq = int_ok ? -0x40000000 : 0;
            }
        }
        const uint64_t qmask = __ballot(hasq);
        // residual-norm band: lane j < nq holds its query's |q - c| and threshold
        float l1_dqc = 0.0f;
        double l1_tau = -1.0;  // lanes without a query skip every tile
        if (a.use_l1 && active && hasq && g == 0) {
            const int pj = start + gq * kWaveQ + j;
            l1_dqc = a.pair_dqc[pj];
            l1_tau = a.tau[a.pair_qid[pj]];
        }
        // the float test's constants and the query ids wait in LDS for the rare path and flush
        if (active && lane < kWaveQ) {
            s_sqid[wid][lane] = q;
            s_qf[wid][lane] = qf;
        }

        // ---- survivor queue (entries li << 4 | query slot) ----
        int nsq = 0;
        auto flush = [&]() {
            for (int e = lane; e < nsq; e += kWave) atomicAdd(&s_scnt[wid][s_sq[wid][e] & 15u], 1);
            __builtin_amdgcn_wave_barrier();
            if (lane < kWaveQ) {
                const int c = s_scnt[wid][lane];
                s_sbase[wid][lane] = c ? atomicAdd(&a.cand_cnt[s_sqid[wid][lane]], c) : 0;
                s_scnt[wid][lane] = 0;
            }
            __builtin_amdgcn_wave_barrier();
            for (int e = lane; e < nsq; e += kWave) {
                const uint32_t ent = s_sq[wid][e];
                const int jj = (int)(ent & 15u);
                const int slot = s_sbase[wid][jj] + atomicAdd(&s_scnt[wid][jj], 1);
                if (slot < a.cap)
                    a.cand_id[(size_t)s_sqid[wid][jj] * a.cap + slot] = v0 + (int)(ent >> 4);
            }
            __builtin_amdgcn_wave_barrier();
            if (lane < kWaveQ) s_scnt[wid][lane] = 0;
            if (a.stats) st_surv += (unsigned long long)nsq;
            nsq = 0;
            // wide ring: the block waits count only the ring's loads, so the stores drain here
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        };

        // ---- rare: queue a tile's passes (rows row0 + r of this lane, r < 4).  The integer
        // test is implied by the exact condition, so nothing is lost, and it passes hardly more
        // rows than the float test would (refinement decides); rows past the slice never pass
        // (thr = INT_MAX, and |acc + kq| < 2^31 - 1), the row check only makes that explicit.
        auto queue = [&](const uint64_t (&sm)[4], int row0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool pass = hasq && ((sm[r] >> lane) & 1ull) && row0 + r < ve;
                const uint64_t pm = __ballot(pass);
                if (pm == 0ull) continue;
                if (nsq + __popcll(pm) > kLbQ) flush();
                if (pass) {
                    const int idx = __builtin_amdgcn_mbcnt_hi(
                        (uint32_t)(pm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)pm, 0u));
                    s_sq[wid][nsq + idx] = ((uint32_t)(row0 + r) << 4) | (uint32_t)j;
                }
                nsq += __popcll(pm);
            }
        };

        // ---- this wave's share of the 64-dim steps of the block's one tile (as in
        // ub_scan_kernel); the replica with rr = 0 carries kq, so the partial sums add up to
        // acc + kq ----
        auto wide_partial = [&](int buf, int (&S)[4], auto r_c) {
            constexpr int RC = decltype(r_c)::value, NS = (KS + RC - 1) / RC;
            const uint4* blk = s_codes[buf];
            v4i A[NS];
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                const int ks = RC == 1 ? i : min(rr + i * RC, KS - 1);
                const uint4 v = blk[(ks * 4 + g) * BV + j];
                A[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
            const int k0 = (RC == 1 || rr == 0) ? kq : 0;
            v4i acc_hi = {0, 0, 0, 0}, acc_lo = {k0, k0, k0, k0};
#pragma unroll
            for (int i = 0; i < NS; ++i) {
                acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], bhi[i], acc_hi, 0, 0, 0);
                acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[i], blo[i], acc_lo, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) S[r] = (acc_hi[r] << 8) + acc_lo[r];
        };
        // the tests of the tile lambda's epilogue on whole sums: thresholds of block buffer
        // tb, row scalars of buffer abuf
        auto wide_judge = [&](const int (&S)[4], int tb, int abuf, int li0) {
            uint64_t sm[4];
            if (int_ok) {
                const int4 th = *reinterpret_cast<const int4*>(&s_thr[tb][wid][4 * g]);
                sm[0] = __ballot(S[0] >= th.x);
                sm[1] = __ballot(S[1] >= th.y);
                sm[2] = __ballot(S[2] >= th.z);
                sm[3] = __ballot(S[3] >= th.w);
            } else {
                const float4 A4 = *reinterpret_cast<const float4*>(&s_A[abuf][4 * g]);
                const float4 r4 = *reinterpret_cast<const float4*>(&s_r[abuf][4 * g]);
                const float Av[4] = {A4.x, A4.y, A4.z, A4.w}, rv[4] = {r4.x, r4.y, r4.z, r4.w};
                const float4 c = s_qf[wid][j];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sm[r] = __ballot(li0 + 4 * g + r < ve &&
                                     fmaf(c.y, rv[r], fmaf(-rv[r], rv[r], Av[r])) <=
                                         fmaf(c.x, (float)S[r], c.z));
            }
            if (((sm[0] | sm[1] | sm[2] | sm[3]) & qmask) == 0ull) return;
            queue(sm, li0 + 4 * g);
        };
        auto wide_finish = [&](int b, int abuf) {
            if (((b & (R - 1)) != rr)) return;
            int S[4] = {0, 0, 0, 0};
            for (int r2 = 0; r2 < R; ++r2) {
                const int4 p = s_part[b & 1][gq * R + r2][lane];
                S[0] += p.x;
                S[1] += p.y;
                S[2] += p.z;
                S[3] += p.w;
            }
            wide_judge(S, b & 1, abuf, vb + b * BV);
        };

        // ---- stream the slice through LDS in 16-vector blocks ----
        const uint4* cells_c = a.cells + (size_t)t0 * G16 * T;  // cluster's first tile
        int ct = vb / T, cw = vb - ct * T;  // tile and slot of the next block to load
        auto gload = [&](int buf, int abuf, int blk0) {
            load_code_block16<KS>(cells_c + (size_t)ct * G16 * T + (size_t)cw * G16, G16, wid,
                                  lane, s_codes[buf], a.vec_Ar + v0, blk0, ve - 1, s_A[abuf],
                                  s_r[abuf]);
            cw += BV;
            if (cw == T) {
                cw = 0;
                ++ct;
            }
        };
        const int nblk = (ve - vb + BV - 1) / BV;
        {
            // ring and replica finish as in ub_scan_kernel
            const int nload = (KS - wid + 3) / 4 + (wid == 0 ? 2 : 0);
            for (int p = 0; p < kWideAhead && p < nblk; ++p) gload(p, p, vb + p * BV);
            int cs = 0;             // b % NBC
            bool band_prev = false;  // block b - 1 was scanned (its deferred finish is due)
            for (int b = 0; b < nblk; ++b) {
                wait_vmcnt(min(kWideAhead - 1, nblk - 1 - b) * nload);
                __syncthreads();
                if (tid == 0 && b == max(nblk - 2, 0)) nxt = atomicAdd(ctr, 1);
                const int blk0 = vb + b * BV;
                if (b + kWideAhead < nblk)
                    gload(cs == 0 ? NBC - 1 : cs - 1, (b + kWideAhead) & 7,
                          blk0 + kWideAhead * BV);
                bool band = active;  // the wave's queries reach the block's tile
                if (a.use_l1 && active) {
                    const float* rm = a.tile_rmm + 2 * (size_t)(t0 + blk0 / T);
                    band = __ballot(l1_tau >= 0.0 && !l1_skips(l1_dqc, l1_tau, rm[0], rm[1])) != 0ull;
                }
                if (active) {
                    // band is the same for the replica waves of a query group (same queries)
                    if (band && int_ok && lane < BV) {
                        const float A = s_A[b & 7][lane], r = s_r[b & 7][lane];
                        s_thr[b & 1][wid][lane] =
                            blk0 + lane < ve ? lb_thr(A, r, tqw, inv_c1w) : INT_MAX;
                    }
                    int S[4];
                    if (R == 1) {
                        if (band) {
                            wide_partial(cs, S, std::integral_constant<int, 1>{});
                            wide_judge(S, b & 1, b & 7, blk0);
                        }
                    } else {
                        if (band) {
                            if (R == 2) wide_partial(cs, S, std::integral_constant<int, 2>{});
                            else wide_partial(cs, S, std::integral_constant<int, 4>{});
                            s_part[b & 1][wid][lane] = make_int4(S[0], S[1], S[2], S[3]);
                        }
                        if (b > 0 && band_prev) wide_finish(b - 1, (b - 1) & 7);
                    }
                }
                band_prev = band;
                cs = cs + 1 == NBC ? 0 : cs + 1;
            }
            if (R > 1 && nblk > 0) {
                __syncthreads();
                if (active && band_prev) wide_finish(nblk - 1, (nblk - 1) & 7);
            }
        }
        if (a.stats && active && rr == 0)
            st_cand += (unsigned long long)nq * (unsigned long long)(ve - vb);
        if (nsq > 0) flush();
        if (tid == 0) s_unit[(it + 1) & 1] = nblk > 0 ? nxt : atomicAdd(ctr, 1);
    }

    if (a.stats && lane == 0) {
        const int slot = (int)(blockIdx.x % kStatSlots) * 4;
        atomicAdd(&a.stats[slot + 0], st_cand);
        atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)(a.D_pad));
        atomicAdd(&a.stats[slot + 2], st_surv);
    }
}

template __global__ void lb_scan_wide_kernel<5>(BatchArgs);
template __global__ void lb_scan_wide_kernel<6>(BatchArgs);
template __global__ void lb_scan_wide_kernel<7>(BatchArgs);
template __global__ void lb_scan_wide_kernel<8>(BatchArgs);
template __global__ void lb_scan_wide_kernel<9>(BatchArgs);
template __global__ void lb_scan_wide_kernel<10>(BatchArgs);
template __global__ void lb_scan_wide_kernel<11>(BatchArgs);
template __global__ void lb_scan_wide_kernel<12>(BatchArgs);
template __global__ void lb_scan_wide_kernel<13>(BatchArgs);
template __global__ void lb_scan_wide_kernel<14>(BatchArgs);
template __global__ void lb_scan_wide_kernel<15>(BatchArgs);
template __global__ void lb_scan_wide_kernel<16>(BatchArgs);

// tau_sq output of the batched route: the seeded float64 threshold, rounded up to float32.
__global__ void tau_to_f32_kernel(const double* tau, float* out, int B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) out[i] = __double2float_ru(tau[i]);
}

}  // namespace trident
