// Cluster-major exact scan (mode 10) on the float32 matrix cores, for gfx950.
//
// The reference's CM-FP32 (src/trident_v4_kernels.cu:268-374) gives every (query, cluster) pair
// one block that walks the cluster's float32 rows with one warp per row, and keeps a per-pair
// top-K in shared memory.  Here a work unit is one slice of a cluster (whole 64-vector blocks)
// and up to 64 of the queries that probe it (the batched route's units), so each row block is
// read from HBM once per 64 queries, and the query x vector products are dense 16 x 16 tiles on
// v_mfma_f32_16x16x4f32: queries are the A rows (held in registers), vectors the B columns (read
// from a padded LDS copy of the block), four independent accumulator chains per tile.
//
// Exactness.  For float32 vectors q, x (exact reals), d = |q - x|^2 = nq + nx - 2 q.x with
// nq = |q|^2, nx = |x|^2:
//   s   = the matrix-core float32 dot product in any association (the chains are summed at the
//         end): each product and addition has relative error <= 2^-23 (round to nearest gives
//         2^-24; the factor two also covers truncation), so |s - q.x| <= kappa sum |q_d x_d|
//         <= kappa |q| |x| with kappa = (D_pad + 8) 2^-23 (1 + 2^-10) (recursive-summation bound
//         over at most D_pad + 8 roundings on any path, first order plus its second-order rest);
//   nq, nx are float64 sums of exact float64 squares (relative error <= D_pad 2^-53 < 2^-43),
//         rounded to float32 (2^-24 more);
//   base = (nq + nx) - 2 s in float32: two roundings, <= 2^-24 (nq + nx) + 2^-24 |base|;
//   the canonical float64 distance d64 of the refine is within 2^-43 d of d.
// With S = nq + nx + 2 |s| (>= |base|, >= d) these add up to <= 2 kappa |q|^ |x|^ + 2^-21 S
// (|.|^ the norms rounded up).  E = (2 kappa |q|^ |x|^ + 2^-20 S) (1 + 2^-20), computed in
// float32, also covers its own roundings and those of base - E and base + E (each <= 2^-24
// (S + E)), so lb = max(base - E, 0) <= d64 <= base + E = ub.
//
// Threshold.  Per query, ub_best holds a float32 value t such that at least K distinct probed
// rows have ub <= t (so the K-th smallest d64 is <= t).  Each lane keeps, for each of its query
// rows, the smallest ub of its column over the unit so far (column j of every tile: distinct
// vectors); when at least K of a row's 16 column minima are below the query's current t, t drops
// to their K-th smallest (atomicMin on the float bits, which order like the values for
// non-negative floats).  After such a drop only K - 1 minima are below t, so the selection runs
// again only when another column's minimum falls below t.  A row is listed iff its lb
// is <= the query's t at that moment; every row of the exact top-K (ties included) qualifies,
// because lb <= d64 <= the K-th smallest d64 <= t.  The listed (lb, ub) keys then give tau = the
// K-th smallest listed ub (fine_tau_kernel), and the refine computes the canonical distance of
// the listed rows whose lb <= tau only.
//
// K > 16.  Sixteen column minima cannot certify K rows, so the in-scan selection never fires;
// instead the warm-up launch over the first probes lists every row, and cm_seed_kernel sets
// ub_best to the K-th smallest listed ub (K distinct probed rows have ub <= it) and empties the
// lists before the main launch, which lists against that fixed threshold.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace trident {

typedef float v4f __attribute__((ext_vector_type(4)));

namespace {

constexpr int kCmBV = 64;  // vectors per LDS block
constexpr int kCmQW = 16;  // queries per wave (matrix rows)

// Loads n floats of src (n <= 4, 16-byte aligned when n == 4 and vec) into v, zero beyond n.
__device__ __forceinline__ float4 load_upto4(const float* src, int n, bool vec) {
    if (n >= 4 && vec) return *reinterpret_cast<const float4*>(src);
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (n > 0) v.x = src[0];
    if (n > 1) v.y = src[1];
    if (n > 2) v.z = src[2];
    if (n > 3) v.w = src[3];
    return v;
}

// The wave's query rows as one lane sees them: rows 4 g + r of its 16-query group.
struct CmRows {
    int rq[4];       // query ids (-1: no query)
    float t_row[4];  // thresholds (-1: never listed)
    float nq_r[4];   // |q| rounded up
    float qn_r[4];   // |q|^2 in float32
    float cmin[4];   // the smallest ub of this lane's column over the unit so far
};

// One 16-vector tile's bounds, thresholds and listing, from its float32 dot products sv (rows
// 4 g + r, column j = lane & 15 = block row bi): lb <= d64 <= ub by the error band above, the
// query's threshold lowered to the K-th smallest of its 16 column minima when at least K are
// below it (K <= 16), and the rows with lb <= threshold listed as (lb, ub) keys.
__device__ __forceinline__ void cm_tile_epilogue(const BatchArgs& a, const v4f sv, int bi, int nvb,
                                                 const float* s_xn, const float* s_nx, float kap2,
                                                 CmRows& Q, int row0,
                                                 unsigned long long& st_surv) {
    const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    const int K = a.K;
    const bool vv = bi < nvb;
    const float xn = s_xn[bi], nx = s_nx[bi];
    float lbf[4], ubf[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float sd = sv[r];
        const float base = (Q.qn_r[r] + xn) - 2.0f * sd;
        const float S = (Q.qn_r[r] + xn) + 2.0f * fabsf(sd);
        const float E = fmaf(kap2 * Q.nq_r[r], nx, 0x1p-20f * S) * (1.0f + 0x1p-20f);
        float lb = fmaxf(base - E, 0.0f), ub = base + E;
        if (!(ub < INFINITY)) {  // overflow or NaN: no bound
            lb = 0.0f;
            ub = INFINITY;
        }
        lbf[r] = vv ? lb : INFINITY;
        ubf[r] = vv ? ub : INFINITY;
        Q.cmin[r] = fminf(Q.cmin[r], ubf[r]);
    }
    // ---- thresholds: the K-th smallest column minimum per query row, when at least K of the
    // row's 16 are below the query's t ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint64_t bm = __ballot(Q.cmin[r] < Q.t_row[r]);
        const int cg = __popcll((bm >> (16 * g)) & 0xffffull);
        if (__ballot(cg >= K) == 0ull) continue;
        const float my = Q.cmin[r];
        int rank = 0;
#pragma unroll 1
        for (int o = 1; o < 16; ++o) {  // rare: kept rolled (no hoisted lane maps)
            const float ot = __shfl_xor(my, o, kWave);
            rank += (ot < my || (ot == my && (j ^ o) < j)) ? 1 : 0;
        }
        float kth = rank == K - 1 ? my : 0.0f;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) kth = fmaxf(kth, __shfl_xor(kth, o, kWave));
        if (cg >= K && Q.rq[r] >= 0 && kth < Q.t_row[r]) {
            Q.t_row[r] = kth;
            if (j == 0) atomicMin(&a.ub_best[Q.rq[r]], __float_as_uint(kth));
        }
    }
    // ---- list the rows with lb <= t: one atomic per (row, lane group); the warm-up pass
    // (cm_emit = 0) only sets thresholds ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if (!a.cm_emit) break;
        // vv explicitly: a query without a threshold yet has t = +inf, and the +inf keys of
        // columns past the slice would compare <= it
        const bool ps = vv && lbf[r] <= Q.t_row[r];
        const uint64_t m = __ballot(ps);
        if (m == 0ull) continue;
        const uint32_t gm = (uint32_t)(m >> (16 * g)) & 0xffffu;
        const int rk = __popc(gm & ((1u << j) - 1u));
        const int leader = gm ? __ffs(gm) - 1 : 0;
        int base = 0;
        if (ps && rk == 0) base = atomicAdd(&a.cand_cnt[Q.rq[r]], __popc(gm));
        base = __shfl(base, 16 * g + leader, kWave);
        if (ps) {
            const int slot = base + rk;
            if (slot < a.cap) {
                const size_t o = (size_t)Q.rq[r] * a.cap + slot;
                a.cand_key[o] = ((uint64_t)__float_as_uint(lbf[r]) << 32) | __float_as_uint(ubf[r]);
                a.cand_id[o] = row0 + bi;
            }
            ++st_surv;
        }
    }
}

}  // namespace

template <int D4>
__global__ __launch_bounds__(256) void cm_scan_kernel(BatchArgs a) {
    constexpr int DP = 4 * D4;  // D_pad
    constexpr int RS = DP + 4;  // LDS row stride: an odd number of 16-byte chunks, so the 16
                                // rows a lane group reads at one offset sit in 16 bank groups
    static_assert(D4 % 8 == 0 && D4 <= 64, "D_pad a multiple of 32, at most 256");
    __shared__ __align__(16) float s_x[kCmBV * RS];
    __shared__ float s_xn[kCmBV];
    __shared__ float s_nx[kCmBV];
    __shared__ double s_qn[kWavesPerBlock][kCmQW];
    __shared__ float s_nq[kWavesPerBlock][kCmQW];
    __shared__ int s_qid[kWavesPerBlock][kCmQW];
    __shared__ int s_unit[2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int D = a.D;
    const int u0 = a.unit_off[a.unit_beg], u1 = min(a.unit_off[a.unit_end], a.max_units);
    const float kap2 = (float)(2.0 * (double)(DP + 8) * 0x1p-23 * (1.0 + 0x1p-10));
    const bool xvec = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(a.xb) & 15) == 0;
    const bool qvec = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(a.xq) & 15) == 0;
    unsigned long long st_cand = 0, st_surv = 0;

    // padding columns [D, DP) stay zero: the blocks rewrite columns [0, D) only
    if (D < DP)
        for (int i = tid; i < kCmBV * (DP - D); i += kBlock)
            s_x[(i / (DP - D)) * RS + D + i % (DP - D)] = 0.0f;

    // work units from one counter (slot (it + 1) & 1 is written while slot it & 1 is read; the
    // previous read of the written slot happened before this iteration's first barrier)
    if (tid == 0) s_unit[0] = atomicAdd(a.ctr, 1);
    for (int it = 0;; ++it) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + u0;
        if (ui < u0 || ui >= u1) break;
        if (tid == 0) s_unit[(it + 1) & 1] = atomicAdd(a.ctr, 1);
        const int4 un = a.units[ui];
        const int cid = un.x & 0xfffff, cnt = un.x >> 20, start = un.y, vb = un.z, ve = un.w;
        const int v0 = a.vec_off[cid];
        const int G = (cnt + kCmQW - 1) / kCmQW;  // 16-query groups (1..4)
        const int R = kWavesPerBlock / G;         // waves sharing a group split its tiles
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(kCmQW, cnt - gq * kCmQW) : 0;
        // rows this unit reads from a host-mapped base: its slice, once
        if (a.host_rows && a.xb_host && tid == 0) atomicAdd(a.host_rows, (unsigned long long)(ve - vb));

        // ---- this wave's queries: A operands (row j, dims g D4 .. g D4 + D4 - 1) and norms ----
        // (initialised on every path: nothing is carried from the previous unit)
        float qa[D4];
#pragma unroll
        for (int k = 0; k < D4; ++k) qa[k] = 0.0f;
        CmRows qs;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            qs.rq[r] = -1;
            qs.t_row[r] = -1.0f;
            qs.nq_r[r] = qs.qn_r[r] = 0.0f;
            qs.cmin[r] = INFINITY;
        }
        if (active) {
            const bool qv = j < nq;
            const int qid = qv ? a.pair_qid[start + gq * kCmQW + j] : 0;
            const float* qp = a.xq + (size_t)qid * D + g * D4;
            double qn = 0.0;
#pragma unroll
            for (int k = 0; k < D4 / 4; ++k) {
                const int left = qv ? D - (g * D4 + 4 * k) : 0;
                const float4 v = load_upto4(qp + 4 * k, left, qvec);
                qa[4 * k] = v.x;
                qa[4 * k + 1] = v.y;
                qa[4 * k + 2] = v.z;
                qa[4 * k + 3] = v.w;
                qn = fma((double)v.x, (double)v.x, qn);
                qn = fma((double)v.y, (double)v.y, qn);
                qn = fma((double)v.z, (double)v.z, qn);
                qn = fma((double)v.w, (double)v.w, qn);
            }
            qn += shfl_f64(qn, lane ^ 16);
            qn += shfl_f64(qn, lane ^ 32);
            if (g == 0) {
                s_qn[wid][j] = qn;
                s_nq[wid][j] = __double2float_ru(sqrt(qn) * (1.0 + 0x1p-40));
                s_qid[wid][j] = qv ? qid : -1;
            }
            wave_sync();
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * g + r;
                qs.rq[r] = row < nq ? s_qid[wid][row] : -1;
                qs.qn_r[r] = (float)s_qn[wid][row];
                qs.nq_r[r] = s_nq[wid][row];
                qs.t_row[r] = qs.rq[r] >= 0 ? __uint_as_float(a.ub_best[qs.rq[r]]) : -1.0f;  // -1: never
            }
        }

        for (int blk0 = vb; blk0 < ve; blk0 += kCmBV) {
            const int nvb = min(kCmBV, ve - blk0);
            // ---- stage the block's rows (columns [0, D)), zero rows past the slice ----
            {
                // chunk i = tid + kBlock k < 64 ceil(D / 4) <= 64 D4, in two halves whose loads
                // are all issued before their LDS stores (two memory round trips per block)
                const int n4 = (D + 3) >> 2;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float4 v[D4 / 8];
#pragma unroll
                    for (int k = 0; k < D4 / 8; ++k) {
                        const int i = tid + kBlock * (h * (D4 / 8) + k);
                        const int r = i / n4, c = i - r * n4;
                        const int left = i < kCmBV * n4 && r < nvb ? D - 4 * c : 0;
                        v[k] = load_upto4(a.xb + (size_t)(v0 + blk0 + min(r, nvb - 1)) * D + 4 * c,
                                          min(left, 4), xvec);
                    }
#pragma unroll
                    for (int k = 0; k < D4 / 8; ++k) {
                        const int i = tid + kBlock * (h * (D4 / 8) + k);
                        const int r = i / n4, c = i - r * n4;
                        // 4 c + 4 <= D_pad (a multiple of 4): columns past D get zeros
                        if (i < kCmBV * n4) *reinterpret_cast<float4*>(s_x + r * RS + 4 * c) = v[k];
                    }
                }
            }
            __syncthreads();
            // ---- row norms in float64: 4 threads a row ----
            {
                const int r = tid >> 2, p = tid & 3;
                const float* xr = s_x + r * RS + p * D4;
                double xn = 0.0;
#pragma unroll 8
                for (int d = 0; d < D4; ++d) xn = fma((double)xr[d], (double)xr[d], xn);
                xn += shfl_f64(xn, lane ^ 1);
                xn += shfl_f64(xn, lane ^ 2);
                if (p == 0) {
                    s_xn[r] = (float)xn;
                    s_nx[r] = __double2float_ru(sqrt(xn) * (1.0 + 0x1p-40));
                }
            }
            __syncthreads();
            if (active) {
                // other units may have lowered the thresholds (four loads in flight, rows
                // without a query read query 0 and keep t = -1)
                uint32_t tb[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) tb[r] = a.ub_best[max(qs.rq[r], 0)];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (qs.rq[r] >= 0) qs.t_row[r] = fminf(qs.t_row[r], __uint_as_float(tb[r]));
                // ---- the wave's tiles: rr, rr + R, ... (16 vectors each), one at a time ----
#pragma unroll 1
                for (int tl = rr; tl < kCmBV / 16 && 16 * tl < nvb; tl += R) {
                    const float* xr = s_x + (16 * tl + j) * RS + g * D4;
                    // four accumulator chains (k-step 4 s4 + k -> chain k), summed at the end
                    v4f acc[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    float4 b = *reinterpret_cast<const float4*>(xr);
#pragma unroll
                    for (int s4 = 0; s4 < D4 / 4; ++s4) {
                        // one step of LDS reads in flight ahead of the matrix cores
                        const float4 bn = *reinterpret_cast<const float4*>(
                            xr + 4 * (s4 + 1 < D4 / 4 ? s4 + 1 : s4));
                        acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4], b.x, acc[0], 0, 0, 0);
                        acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 1], b.y, acc[1], 0, 0, 0);
                        acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 2], b.z, acc[2], 0, 0, 0);
                        acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 3], b.w, acc[3], 0, 0, 0);
                        b = bn;
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    // VALU reads of matrix-core results: wait states fenced from the scheduler
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("s_nop 7\n\ts_nop 7");
                    __builtin_amdgcn_sched_barrier(0);
                    const v4f sv = (acc[0] + acc[1]) + (acc[2] + acc[3]);
                    cm_tile_epilogue(a, sv, 16 * tl + j, nvb, s_xn, s_nx, kap2, qs, v0 + blk0, st_surv);
                }
                if (a.stats && rr == 0 && lane == 0) st_cand += (unsigned long long)nq * nvb;
            }
            __syncthreads();  // the next block overwrites s_x, s_xn, s_nx
        }
    }

    if (a.stats) {
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) st_surv += __shfl_xor(st_surv, o, kWave);
        if (lane == 0) {
            const int slot = (int)(blockIdx.x % kStatSlots) * 4;
            atomicAdd(&a.stats[slot + 0], st_cand);
            atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)DP);
            atomicAdd(&a.stats[slot + 2], st_surv);
        }
    }
}

// Wide layout (D_pad > 256, up to 1024): a query row no longer fits in registers, so the
// dimensions are walked in chunks of kCmWC dims.  Per 64-row block and chunk the block's rows
// are staged in LDS (64 x kCmWC floats, 33 KB: four workgroups per CU) and each wave reloads its
// 16 query rows' chunk (kCmWC / 4 floats a lane, from L2); every tile of the wave keeps one
// accumulator chain across the chunks (the wave's up to four tiles are independent chains for
// the matrix core).  The float64 row norms add up chunk by chunk in LDS.  Bounds, thresholds and
// listing are those of the narrow kernel, with kappa over the padded dimensions.
constexpr int kCmWC = 128;

__global__ __launch_bounds__(256) void cm_scan_wide_kernel(BatchArgs a) {
    constexpr int C4 = kCmWC / 4;  // floats per lane per chunk
    constexpr int RS = kCmWC + 4;  // LDS row stride: an odd number of 16-byte chunks
    __shared__ __align__(16) float s_x[kCmBV * RS];
    __shared__ double s_xd[kCmBV];
    __shared__ float s_xn[kCmBV];
    __shared__ float s_nx[kCmBV];
    __shared__ double s_qn[kWavesPerBlock][kCmQW];
    __shared__ float s_nq[kWavesPerBlock][kCmQW];
    __shared__ int s_qid[kWavesPerBlock][kCmQW];
    __shared__ int s_unit[2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int D = a.D;
    const int nch = (a.D_pad + kCmWC - 1) / kCmWC;  // chunks; dims past D are zero
    const int u0 = a.unit_off[a.unit_beg], u1 = min(a.unit_off[a.unit_end], a.max_units);
    const float kap2 = (float)(2.0 * (double)(nch * kCmWC + 8) * 0x1p-23 * (1.0 + 0x1p-10));
    const bool xvec = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(a.xb) & 15) == 0;
    const bool qvec = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(a.xq) & 15) == 0;
    unsigned long long st_cand = 0, st_surv = 0;

    if (tid == 0) s_unit[0] = atomicAdd(a.ctr, 1);
    for (int it = 0;; ++it) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + u0;
        if (ui < u0 || ui >= u1) break;
        if (tid == 0) s_unit[(it + 1) & 1] = atomicAdd(a.ctr, 1);
        const int4 un = a.units[ui];
        const int cid = un.x & 0xfffff, cnt = un.x >> 20, start = un.y, vb = un.z, ve = un.w;
        const int v0 = a.vec_off[cid];
        const int G = (cnt + kCmQW - 1) / kCmQW;  // 16-query groups (1..4)
        const int R = kWavesPerBlock / G;         // waves sharing a group split its tiles
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(kCmQW, cnt - gq * kCmQW) : 0;
        // rows this unit reads from a host-mapped base: its slice, once
        if (a.host_rows && a.xb_host && tid == 0) atomicAdd(a.host_rows, (unsigned long long)(ve - vb));
        const bool qv = j < nq;
        const int qid = active && qv ? a.pair_qid[start + gq * kCmQW + j] : 0;
        const float* qrow = a.xq + (size_t)qid * D;

        // ---- this wave's query rows: norms over all dims (lane (j, g): dims c kCmWC + g C4
        // .. + C4 - 1 of query j, for every chunk c) ----
        CmRows qs;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            qs.rq[r] = -1;
            qs.t_row[r] = -1.0f;
            qs.nq_r[r] = qs.qn_r[r] = 0.0f;
            qs.cmin[r] = INFINITY;
        }
        if (active) {
            double qn = 0.0;
            for (int c = 0; c < nch; ++c) {
#pragma unroll
                for (int k = 0; k < C4 / 4; ++k) {
                    const int d0 = c * kCmWC + g * C4 + 4 * k;
                    const float4 v = load_upto4(qrow + d0, qv ? D - d0 : 0, qvec);
                    qn = fma((double)v.x, (double)v.x, qn);
                    qn = fma((double)v.y, (double)v.y, qn);
                    qn = fma((double)v.z, (double)v.z, qn);
                    qn = fma((double)v.w, (double)v.w, qn);
                }
            }
            qn += shfl_f64(qn, lane ^ 16);
            qn += shfl_f64(qn, lane ^ 32);
            if (g == 0) {
                s_qn[wid][j] = qn;
                s_nq[wid][j] = __double2float_ru(sqrt(qn) * (1.0 + 0x1p-40));
                s_qid[wid][j] = qv ? qid : -1;
            }
            wave_sync();
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * g + r;
                qs.rq[r] = row < nq ? s_qid[wid][row] : -1;
                qs.qn_r[r] = (float)s_qn[wid][row];
                qs.nq_r[r] = s_nq[wid][row];
                qs.t_row[r] = qs.rq[r] >= 0 ? __uint_as_float(a.ub_best[qs.rq[r]]) : -1.0f;
            }
        }

        for (int blk0 = vb; blk0 < ve; blk0 += kCmBV) {
            const int nvb = min(kCmBV, ve - blk0);
            // the wave's tiles rr, rr + R, ... inside the block (1 to 4, wave-uniform), one
            // accumulator chain each
            int nt = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) nt += t * R < kWavesPerBlock && 16 * (rr + t * R) < nvb ? 1 : 0;
            v4f acc[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            for (int c = 0; c < nch; ++c) {
                const int cb = c * kCmWC;
                // ---- stage the block's rows, dims [cb, cb + kCmWC) (zero past D): 64 x 32
                // float4 chunks, eight per thread, in two halves whose loads are all issued
                // before their LDS stores ----
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float4 v[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int i = tid + kBlock * (4 * h + k);
                        const int r = i / (kCmWC / 4), c4 = i - r * (kCmWC / 4);
                        const int d0 = cb + 4 * c4;
                        v[k] = load_upto4(a.xb + (size_t)(v0 + blk0 + min(r, nvb - 1)) * D + d0,
                                          min(r < nvb ? D - d0 : 0, 4), xvec);
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int i = tid + kBlock * (4 * h + k);
                        const int r = i / (kCmWC / 4), c4 = i - r * (kCmWC / 4);
                        *reinterpret_cast<float4*>(s_x + r * RS + 4 * c4) = v[k];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // ---- this chunk's query values (A operands; a lane's dims lie wholly inside
                // or outside D when D % 4 == 0, the vector path) ----
                float qa[C4];
                if (active) {
#pragma unroll
                    for (int k = 0; k < C4 / 4; ++k) {
                        const int d0 = cb + g * C4 + 4 * k;
                        const int left = qv ? D - d0 : 0;
                        float4 v;
                        if (qvec) v = left > 0 ? *reinterpret_cast<const float4*>(qrow + d0)
                                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        else v = load_upto4(qrow + d0, left, false);
                        qa[4 * k] = v.x;
                        qa[4 * k + 1] = v.y;
                        qa[4 * k + 2] = v.z;
                        qa[4 * k + 3] = v.w;
                    }
                }
                __syncthreads();
                __builtin_amdgcn_sched_barrier(0);
                // ---- the chunk's share of the row norms: 4 threads a row ----
                {
                    const int r = tid >> 2, p = tid & 3;
                    const float* xr = s_x + r * RS + p * C4;
                    double xn = 0.0;
#pragma unroll 8
                    for (int d = 0; d < C4; ++d) xn = fma((double)xr[d], (double)xr[d], xn);
                    xn += shfl_f64(xn, lane ^ 1);
                    xn += shfl_f64(xn, lane ^ 2);
                    if (p == 0) s_xd[r] = (c == 0 ? 0.0 : s_xd[r]) + xn;
                }
                __builtin_amdgcn_sched_barrier(0);
                if (active) {
                    // NT tiles (rows 16 (rr + t R) ..), straight-line per 4-dim step
                    auto mma = [&](auto nt_c) __attribute__((always_inline)) {
                        constexpr int NT = decltype(nt_c)::value;
#pragma unroll
                        for (int s4 = 0; s4 < C4 / 4; ++s4) {
                            float4 b[NT];
#pragma unroll
                            for (int t = 0; t < NT; ++t)
                                b[t] = *reinterpret_cast<const float4*>(
                                    s_x + (16 * (rr + t * R) + j) * RS + g * C4 + 4 * s4);
#pragma unroll
                            for (int t = 0; t < NT; ++t) {
                                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4], b[t].x, acc[t], 0, 0, 0);
                                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 1], b[t].y, acc[t], 0, 0, 0);
                                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 2], b[t].z, acc[t], 0, 0, 0);
                                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + 3], b[t].w, acc[t], 0, 0, 0);
                            }
                            // one step's LDS reads at a time: hoisting every step's reads ahead
                            // of the matrix cores would hold them all in registers
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    };
                    switch (nt) {
                        case 1: mma(std::integral_constant<int, 1>{}); break;
                        case 2: mma(std::integral_constant<int, 2>{}); break;
                        case 3: mma(std::integral_constant<int, 3>{}); break;
                        default: mma(std::integral_constant<int, 4>{}); break;
                    }
                }
                __syncthreads();  // the next chunk overwrites s_x; s_xd complete after the last
            }
            if (tid < kCmBV) {
                const double xn = s_xd[tid];
                s_xn[tid] = (float)xn;
                s_nx[tid] = __double2float_ru(sqrt(xn) * (1.0 + 0x1p-40));
            }
            __syncthreads();
            if (active) {
                uint32_t tb[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) tb[r] = a.ub_best[max(qs.rq[r], 0)];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (qs.rq[r] >= 0) qs.t_row[r] = fminf(qs.t_row[r], __uint_as_float(tb[r]));
                // VALU reads of matrix-core results: wait states fenced from the scheduler
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("s_nop 7\n\ts_nop 7");
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (t >= nt) break;
                    cm_tile_epilogue(a, acc[t], 16 * (rr + t * R) + j, nvb, s_xn, s_nx, kap2, qs,
                                     v0 + blk0, st_surv);
                }
                if (a.stats && rr == 0 && lane == 0) st_cand += (unsigned long long)nq * nvb;
            }
            __syncthreads();  // the next block overwrites s_xd, s_xn, s_nx
        }
    }

    if (a.stats) {
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) st_surv += __shfl_xor(st_surv, o, kWave);
        if (lane == 0) {
            const int slot = (int)(blockIdx.x % kStatSlots) * 4;
            atomicAdd(&a.stats[slot + 0], st_cand);
            atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)a.D_pad);
            atomicAdd(&a.stats[slot + 2], st_surv);
        }
    }
}

template __global__ void cm_scan_kernel<8>(BatchArgs);
template __global__ void cm_scan_kernel<16>(BatchArgs);
template __global__ void cm_scan_kernel<24>(BatchArgs);
template __global__ void cm_scan_kernel<32>(BatchArgs);
template __global__ void cm_scan_kernel<40>(BatchArgs);
template __global__ void cm_scan_kernel<48>(BatchArgs);
template __global__ void cm_scan_kernel<56>(BatchArgs);
template __global__ void cm_scan_kernel<64>(BatchArgs);

}  // namespace trident
