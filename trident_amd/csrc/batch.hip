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
//               src/trident_v4_kernels.cu:626-676, computed for 64 queries at once; the K-th
//               smallest upper bound of any K vectors bounds the K-th distance).
// Pass B (LB):  for every probe, vectors whose lower bound passes tau[q] are appended (sorted
//               position) to the query's candidate list.  The test runs in float32 with an
//               additive slack that bounds every rounding of it.
// Refine:       one wave per query computes the canonical float64 distance of each listed
//               survivor and keeps it iff <= tau[q] (the reference's Stage Z, :796-941).
//
// Scheduling: a work unit is (cluster, <= 64 queries, slice of the cluster's vectors); each of
// the workgroup's 4 waves owns 16 of the queries (the MFMA N dimension).  Units of one launch
// are split into 8 contiguous ranges, one per XCD (blockIdx & 7), so a cluster's codes are read
// from HBM once per XCD and then served by that XCD's L2; within a range each workgroup takes
// the next unit from its XCD's counter (persistent grid, one atomic per unit).  The unit's
// vectors stream through LDS in 64-vector blocks, double-buffered: all 256 threads load block
// b+1 (16-byte loads, D_pad/4 rows of 256 contiguous bytes) while the waves run block b from
// LDS, one barrier per block.  Lane l = (i = l & 15, g = l >> 4) holds, for every 64-dim step,
// bytes of dims step*64 + g*16 + [0, 16): vector i's codes in the A operand and query i's
// weights in the B operand (any dim-to-byte assignment shared by A and B computes the same
// contraction); the result row 4g + r, column i sits in lane l, register r.
#include "common.hpp"
#include "kernels.hpp"

namespace trident {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kUbList = 16;  // per-lane upper-bound list (K <= 64)
constexpr int kBlkV = 64;    // vectors per LDS block
constexpr int kWaveQ = 16;   // queries per wave

// Vector slices of a cluster in pass p.  Pass-1 segments (the seeding probes) keep whole
// clusters: the K-th smallest upper bound over a slice is a much weaker threshold than over
// the cluster.  Pass-2 segments are sliced so that no unit runs far longer than the others.
__device__ __forceinline__ int splits_of(int n, int p) {
    if (n <= 0) return 0;
    return p ? min(kMaxSplit, (n + kSplitVec - 1) / kSplitVec) : 1;
}

__device__ __forceinline__ int units_of_entry(const int32_t* seg_off, const int32_t* vec_off,
                                              int nlist, int e) {
    const int p = e >= nlist ? 1 : 0, c = e - p * nlist;
    const int32_t* so = seg_off + p * (nlist + 1);
    const int q = so[c + 1] - so[c];
    const int uq = p ? kUnitQ : kUnitQ0;
    return q > 0 ? ((q + uq - 1) / uq) * splits_of(vec_off[c + 1] - vec_off[c], p) : 0;
}

// grid 1: exclusive scan of the unit counts of the 2 * nlist (pass, cluster) segments.
__global__ __launch_bounds__(256) void unit_scan_kernel(const int32_t* seg_off,
                                                        const int32_t* vec_off, int nlist,
                                                        int32_t* unit_off) {
    __shared__ uint32_t s_wtot[kWavesPerBlock];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int E = 2 * nlist;
    const int per = (E + kBlock - 1) / kBlock;
    const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
    uint32_t local = 0;
    for (int e = e0; e < e1; ++e) local += (uint32_t)units_of_entry(seg_off, vec_off, nlist, e);
    uint32_t inc = local;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = (uint32_t)__shfl_up((int)inc, o, kWave);
        if (lane >= o) inc += t;
    }
    if (lane == kWave - 1) s_wtot[wid] = inc;
    __syncthreads();
    uint32_t run = inc - local, total = 0;
    for (int w = 0; w < kWavesPerBlock; ++w) {
        if (w < wid) run += s_wtot[w];
        total += s_wtot[w];
    }
    for (int e = e0; e < e1; ++e) {
        unit_off[e] = (int32_t)run;
        run += (uint32_t)units_of_entry(seg_off, vec_off, nlist, e);
    }
    if (tid == 0) unit_off[E] = (int32_t)total;
}

// One thread per unit: locate its segment by binary search over unit_off, then its query block
// and vector slice.  Slices start on 64-vector blocks and are never empty (n > 64 S (S - 1)
// whenever S = ceil(n / kSplitVec) > 1).
__global__ __launch_bounds__(256) void unit_fill_kernel(const int32_t* seg_off,
                                                        const int32_t* vec_off, int nlist,
                                                        const int32_t* unit_off, int M1,
                                                        int4* units, int max_units) {
    const int E = 2 * nlist;
    const int total = min(unit_off[E], max_units);
    for (int u = blockIdx.x * blockDim.x + threadIdx.x; u < total; u += gridDim.x * blockDim.x) {
        int lo = 0, hi = E - 1;  // largest e with unit_off[e] <= u
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (unit_off[mid] <= u) lo = mid;
            else hi = mid - 1;
        }
        const int p = lo >= nlist ? 1 : 0, c = lo - p * nlist;
        const int32_t* so = seg_off + p * (nlist + 1);
        const int n = vec_off[c + 1] - vec_off[c];
        const int S = splits_of(n, p);
        const int local = u - unit_off[lo];
        const int qb = local / S, sp = local - qb * S;
        const int q = so[c + 1] - so[c];
        const int uq = p ? kUnitQ : kUnitQ0;
        const int cnt = min(uq, q - qb * uq);
        const int len = ((n + S - 1) / S + kBlkV - 1) & ~(kBlkV - 1);
        const int vb = sp * len, ve = min(n, vb + len);
        units[u] = make_int4(c | (cnt << 20), (p ? M1 : 0) + so[c] + qb * uq, vb, ve);
    }
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

// Exact test of the listed survivors, in place: slot s of query q holds a sorted position on
// entry and (key, original id) on exit, or (kKeyInvalid, kIdInvalid) when the canonical
// float64 distance exceeds tau[q].  One wave per query, one survivor per lane; each lane walks
// its own row in dimension order with 16-byte loads.  An overflowed list (count > cap) is left
// alone: the merge rescans that query's probes exhaustively.
__global__ __launch_bounds__(256) void refine_survivors_kernel(BatchArgs a, int B) {
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    if (q >= B) return;
    const int cnt = a.cand_cnt[q];
    if (cnt > a.cap) return;
    const double tau = a.tau[q];
    const int D = a.D;
    const float* qr = a.xq + (size_t)q * D;
    uint64_t* ck = a.cand_key + (size_t)q * a.cap;
    int32_t* ci = a.cand_id + (size_t)q * a.cap;
    const bool vec4 = (D & 3) == 0 && ((reinterpret_cast<uintptr_t>(a.xb) |
                                         reinterpret_cast<uintptr_t>(a.xq)) & 15) == 0;
    unsigned long long ins = 0;
    for (int s = lane; s < cnt; s += kWave) {
        const int pos = ci[s];
        const float* xr = a.xb + (size_t)pos * D;
        double acc = 0.0;
        if (vec4) {
#pragma unroll 4
            for (int d = 0; d < D; d += 4) {
                const float4 x = *reinterpret_cast<const float4*>(xr + d);
                const float4 y = *reinterpret_cast<const float4*>(qr + d);
                double t = (double)x.x - (double)y.x;
                acc = fma(t, t, acc);
                t = (double)x.y - (double)y.y;
                acc = fma(t, t, acc);
                t = (double)x.z - (double)y.z;
                acc = fma(t, t, acc);
                t = (double)x.w - (double)y.w;
                acc = fma(t, t, acc);
            }
        } else {
            for (int d = 0; d < D; ++d) {
                const double t = (double)xr[d] - (double)qr[d];
                acc = fma(t, t, acc);
            }
        }
        const bool ok = acc <= tau;
        ck[s] = ok ? key_of(acc) : kKeyInvalid;
        ci[s] = ok ? a.orig_ids[pos] : kIdInvalid;
        if (a.stats) ins += __popcll(__ballot(ok));  // lane 0 is active in every round
    }
    if (a.stats && lane == 0 && ins)
        atomicAdd(&a.stats[(q % kStatSlots) * 4 + 3], ins);
}

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

// Waves [0, nlist): per-cluster bounds of the f32 slack, A_max = 255^2 sum delta^2 (>= A_x,
// codes <= 255) and r_max = 2 sqrt(sum eps^2) (>= r_x = |a| + |b| <= 2 |a + b| for the
// non-negative per-dim error terms bounded by eps).  Waves [nlist, nlist + B): per-query
// sum of qerr^2 (the rotation error of q_rot, squared).
__global__ __launch_bounds__(256) void aux_bounds_kernel(BatchArgs a, int nlist, int B,
                                                         double* cbound, double* qep) {
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    const int D_pad = a.D_pad;
    if (wv < nlist) {
        const size_t off = a.per_cluster ? (size_t)wv * D_pad : 0;
        double dd = 0.0, ee = 0.0;
        for (int d = lane; d < D_pad; d += kWave) {
            const double dl = (double)a.delta[off + d], e = (double)a.eps[off + d];
            dd = fma(dl, dl, dd);
            ee = fma(e, e, ee);
        }
        dd = wave_sum_f64(dd);
        ee = wave_sum_f64(ee);
        if (lane == 0) {
            cbound[2 * wv] = 65025.0 * dd * (1.0 + 1e-12);
            cbound[2 * wv + 1] = 2.0 * sqrt(ee) * (1.0 + 1e-12);
        }
    } else if (wv < nlist + B) {
        const double* qe = a.qerr + (size_t)(wv - nlist) * D_pad;
        double ep = 0.0;
        for (int d = lane; d < D_pad; d += kWave) ep = fma(qe[d], qe[d], ep);
        ep = wave_sum_f64(ep);
        if (lane == 0) qep[wv - nlist] = ep;
    }
}

// 16 lanes per grouped pair p (4 pairs per wave): the query's int8 weight planes against its
// cluster's SQ8 grid and the pair's threshold-independent scalars.  Lane l owns dims
// 64 k + 4 l + [0, 4) (coalesced 32-byte row pieces, one packed 32-bit store per plane).
//   w_d = delta_d * (q_rot,d - vmin_d);  s = 2^(ilogb(max |w|) - 14), doubled if max|w|/s >
//   32639, so |w_int| <= 32639;  w_int = rint(w / s) = 256 hi + lo  (hi, lo in [-128, 127]).
// Plane bytes past D_pad (up to DP) are zero, so the scan may read whole 64-dim steps.
template <int KS>
__global__ __launch_bounds__(256) void pair_prep_kernel(BatchArgs a) {
    const int lane = threadIdx.x & 63, l = lane & 15;
    const int p = (blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6)) * 4 + (lane >> 4);
    const bool valid = p < a.M;
    const int pp = valid ? p : a.M - 1;  // out-of-range groups redo the last pair, store nothing
    const int c = a.pair_cid[pp], q = a.pair_qid[pp];
    const int D_pad = a.D_pad, DP = a.DP;
    const size_t off = a.per_cluster ? (size_t)c * D_pad : 0;
    const double* xr = a.xrot64 + (size_t)q * D_pad;
    double w[KS][4];
    double mx = 0.0, Qp = 0.0;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const int d0 = 64 * k + 4 * l;  // D_pad is a multiple of 4: all 4 dims or none
#pragma unroll
        for (int e = 0; e < 4; ++e) w[k][e] = 0.0;
        if (d0 < D_pad) {
            const double2 x01 = *reinterpret_cast<const double2*>(xr + d0);
            const double2 x23 = *reinterpret_cast<const double2*>(xr + d0 + 2);
            const double xv[4] = {x01.x, x01.y, x23.x, x23.y};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double qp = xv[e] - (double)a.vmin[off + d0 + e];
                w[k][e] = (double)a.delta[off + d0 + e] * qp;
                mx = fmax(mx, fabs(w[k][e]));
                Qp = fma(qp, qp, Qp);
            }
        }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx = fmax(mx, shfl_f64(mx, lane ^ o));
    Qp = sum16_f64(Qp);
    // s and 1/s are powers of two (|e| <= 1010 here), so w * (1/s) is exactly w / s
    int es = 0;
    if (mx > 0x1p-100) {
        es = ilogb(mx) - 14;
        if (ldexp(mx, -es) > 32639.0) ++es;
    }
    const double s = ldexp(1.0, es), inv_s = ldexp(1.0, -es);
    double errs = 0.0;
    int wsum = 0, wabs = 0;
    int8_t* hi_p = a.pw + (size_t)pp * 2 * DP;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        uint32_t hw = 0u, lw = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int wi = (int)rint(w[k][e] * inv_s);  // 0 for dims >= D_pad
            errs += fabs(w[k][e] - s * (double)wi) + 0x1p-52 * fabs(w[k][e]);
            wsum += wi;
            wabs += abs(wi);
            const int hi = (wi + 128) >> 8;
            hw |= ((uint32_t)hi & 0xffu) << (8 * e);
            lw |= ((uint32_t)(wi - (hi << 8)) & 0xffu) << (8 * e);
        }
        if (valid) {
            *reinterpret_cast<uint32_t*>(hi_p + 64 * k + 4 * l) = hw;
            *reinterpret_cast<uint32_t*>(hi_p + DP + 64 * k + 4 * l) = lw;
        }
    }
    errs = sum16_f64(errs);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        wsum += __shfl_xor(wsum, o, kWave);
        wabs += __shfl_xor(wabs, o, kWave);
    }
    if (valid && l == 0) {
        PairRec r;
        r.Qp = Qp;
        r.err_q = 255.0 * errs * (1.0 + 0x1p-40);
        r.e_q = sqrt(a.qep[q]) * (1.0 + 1e-12) + 0x1p-52 * sqrt(Qp) + 1e-300;
        r.cW = 128.0 * (double)wsum;
        r.c1 = 2.0 * s;
        r.a_max = a.cbound[2 * c];
        r.r_max = a.cbound[2 * c + 1];
        r.acc_max = 128.0 * (double)wabs;
        a.prec[pp] = r;
    }
}

template __global__ void pair_prep_kernel<1>(BatchArgs);
template __global__ void pair_prep_kernel<2>(BatchArgs);
template __global__ void pair_prep_kernel<3>(BatchArgs);
template __global__ void pair_prep_kernel<4>(BatchArgs);

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

// A 64-vector code block in LDS: 16-byte cell rg * 64 + v holds vector v's codes of dims
// 16 rg .. 16 rg + 15 (code rows 4 rg .. 4 rg + 3, one 32-bit row each) as c' = c - 128, so
// the MFMA A operand of 64 dims is one 16-byte read.  Thread tid moves the cells of vector
// tid & 63, row groups (tid >> 6) + 4 jj: four 4-byte loads, each coalesced over the wave (64
// consecutive vectors of one code row).  D4 is a multiple of 8, so a row group is either
// wholly inside D_pad or wholly past it (then zero).
__device__ __forceinline__ uint4 cell_load(const uint32_t* base, int jj, int tid, int D4, int T) {
    const int r0 = 4 * ((tid >> 6) + 4 * jj);
    if (r0 >= D4) return make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
    const uint32_t* p = base + (size_t)r0 * T + (tid & 63);
    return make_uint4(p[0], p[T], p[2 * T], p[3 * T]);
}

__device__ __forceinline__ void cell_store(uint4* blk, uint4 c, int jj, int tid) {
    blk[((tid >> 6) + 4 * jj) * kBlkV + (tid & 63)] =
        make_uint4(c.x ^ 0x80808080u, c.y ^ 0x80808080u, c.z ^ 0x80808080u, c.w ^ 0x80808080u);
}

template <bool UB_PASS, int KS>
__global__ __launch_bounds__(256) void batch_scan_kernel(BatchArgs a) {
    constexpr int kRows = KS * 16;  // code rows (4 dims each) held per block buffer
    __shared__ uint4 s_codes[2][kRows * kBlkV / 4];
    __shared__ __align__(16) float2 s_ar[2][kBlkV];
    __shared__ float s_ubl[UB_PASS ? kWavesPerBlock : 1][UB_PASS ? kWaveQ * kWave : 1];
    __shared__ int s_unit[2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int total = min(a.unit_off[a.unit_end], a.max_units);
    const int nx = (total + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int rb = xcd * nx, re = min(total, rb + nx);
    int32_t* ctr = a.ctr + xcd * kCtrStride;
    const int D_pad = a.D_pad, D4 = D_pad >> 2, T = a.T;
    unsigned long long st_cand = 0, st_surv = 0;

    for (int it = 0;; ++it) {
        // (s_unit alternates: slot it & 1 is rewritten two barriers after everyone read it)
        if (tid == 0) s_unit[it & 1] = atomicAdd(ctr, 1);
        __syncthreads();
        const int ui = __builtin_amdgcn_readfirstlane(s_unit[it & 1]) + rb;
        if (ui >= re) break;
        const int4 un = a.units[ui];
        const int cid = un.x & 0xfffff, cnt = un.x >> 20, start = un.y, vb = un.z, ve = un.w;
        // The unit's queries form G groups of <= 16; each group gets R = 4 / G waves, which
        // split every block's four 16-vector tiles (replica rr takes tiles rr, rr + R, ...).
        const int G = (cnt + kWaveQ - 1) / kWaveQ;
        const int R = kWavesPerBlock / G;
        const int gq = wid / R, rr = wid - gq * R;
        const bool active = gq < G;
        const int nq = active ? min(kWaveQ, cnt - gq * kWaveQ) : 0;  // this wave's queries
        const bool hasq = j < nq;
        const int v0 = a.vec_off[cid];
        const int t0 = a.tile_off[cid];
        int q = 0;

        // ---- per-query weights for this lane's dims (active waves only) ----
        v4i bhi[KS], blo[KS];
        double e_q = 0.0, c1 = 0.0, cW = 0.0, AQ = 0.0;
        float c1f = 0.0f, c2f = 0.0f, H32 = INFINITY;  // no threshold: every row passes
        if (active) {
            // Prepared by pair_prep_kernel: lane (j, g) takes bytes [ks*64 + g*16, +16) of
            // query j's planes and the pair's scalars.
            const int pj = start + gq * kWaveQ + (hasq ? j : 0);
            q = a.pair_qid[pj];
            const int8_t* hp = a.pw + (size_t)pj * 2 * a.DP + g * 16;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                bhi[ks] = *reinterpret_cast<const v4i*>(hp + ks * 64);
                blo[ks] = *reinterpret_cast<const v4i*>(hp + a.DP + ks * 64);
            }
            const PairRec pr = a.prec[pj];
            const double Qp = pr.Qp, err_q = pr.err_q;
            e_q = pr.e_q;
            cW = pr.cW;
            c1 = pr.c1;
            if constexpr (UB_PASS) {
                AQ = (Qp + 2.0 * err_q) * (1.0 + 1e-13);
            } else {
                const double tau = a.tau[q];
                const double tq = sqrt(tau * a.rot_sq_max) * (1.0 + 1e-12) + e_q;
                if (tq < 1e30) {
                    // Survive iff A - r^2 - 2 tq r <= 2 s dot + 2 err - Q + tq^2 (the norm-form
                    // lower bound against sqrt(tau) scaled to the rotated space).  Evaluated as
                    //   L = fma(c2, r, fma(-r, r, A_lo)) <= R = fma(c1, float(acc), H32)
                    // with acc = dot - 128 sum(w_int) (exact int32), c1 = 2s (a power of two),
                    // c2 <= -2 tq and H32 >= 2 s 128 sum(w_int) + 2 err - Q + tq^2 + slack.
                    // Each of the 4 f32 roundings is at most 2^-24 of a term bounded by
                    //   X = A_max + r_max^2 + 2 tq r_max + c1 acc_max + |H|,
                    // with A_max = 255^2 sum delta^2 (codes <= 255), r_max = 2 sqrt(sum eps^2)
                    // (r_x <= |a| + |b| <= 2 |a + b| for the non-negative per-dim error terms)
                    // and |acc| <= acc_max = 128 sum |w_int|; slack = 2^-22 X covers them all.
                    const double G = 2.0 * err_q - Qp * (1.0 - 1e-13) + tq * tq;
                    const double H = c1 * cW + G;
                    const double X = pr.a_max + pr.r_max * pr.r_max + 2.0 * tq * pr.r_max +
                                     c1 * pr.acc_max + fabs(H);
                    const double slack = 0x1p-22 * X * (1.0 + 1e-6) + 1e-30;
                    H32 = __double2float_ru(H + slack);
                    c1f = (float)c1;
                    c2f = -__double2float_ru(2.0 * tq);
                }
            }
            if (!hasq) H32 = -INFINITY;  // lane has no query: nothing survives
        }

        float ubl[kUbList];
        if constexpr (UB_PASS) {
#pragma unroll
            for (int i = 0; i < kUbList; ++i) ubl[i] = INFINITY;
        }

        // ---- one 16-vector tile of the block in LDS buffer buf ----
        auto tile = [&](int buf, int t, int li0) {
            // A operand: lane (i = j, g) reads vector 16t + i's 16 code bytes of dims
            // ks*64 + g*16 + [0, 16) (row group ks*4 + g), already offset to c' = c - 128.
            const uint4* blk = s_codes[buf];
            v4i A[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 v = blk[(ks * 4 + g) * kBlkV + t * 16 + j];
                A[ks] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
            v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks], bhi[ks], acc_hi, 0, 0, 0);
                acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks], blo[ks], acc_lo, 0, 0, 0);
            }
            // The matrix core does not interlock VALU reads of its results: keep 16 wait
            // states (plus the compiler's own padding) between the last MFMA and the first
            // accumulator read, fenced so the scheduler cannot move either side across.  (The
            // compiler's padding alone fell short when a branch sat between the two: rows read
            // the previous tile's sums.)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_nop 7\n\ts_nop 7");
            __builtin_amdgcn_sched_barrier(0);
            // per-row scalars: (P = A_lo - r^2, r) in the lower-bound pass, (A_lo, r) in the
            // upper-bound pass; rows past the slice hold (NaN, +inf), which neither test accepts
            const float4 ar01 = *reinterpret_cast<const float4*>(&s_ar[buf][t * 16 + 4 * g]);
            const float4 ar23 = *reinterpret_cast<const float4*>(&s_ar[buf][t * 16 + 4 * g + 2]);
            const float Ar[4][2] = {{ar01.x, ar01.y}, {ar01.z, ar01.w}, {ar23.x, ar23.y},
                                    {ar23.z, ar23.w}};
            // epilogue: rows 4g + r (vectors), column j (query); the lower-bound pass keeps
            // each row's survivors as the wave mask its compare produces
            uint64_t sm[4] = {0ull, 0ull, 0ull, 0ull};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int acc = (acc_hi[r] << 8) + acc_lo[r];
                if constexpr (UB_PASS) {
                    const double dot = (double)acc + cW;
                    const double Alo = (double)Ar[r][0], rr = (double)Ar[r][1];
                    const double E = fmax(fma(-c1, dot, Alo * (1.0 + 0x1p-22) + AQ), 0.0);
                    const float s32 = sqrtf((float)(E * (1.0 + 1e-12))) * (1.0f + 0x1p-20f);
                    const float u = (s32 + (float)rr + (float)e_q) * (1.0f + 0x1p-20f);
                    if (u < ubl[kUbList - 1]) {
#pragma unroll
                        for (int i = kUbList - 1; i > 0; --i)
                            ubl[i] = (u < ubl[i - 1]) ? ubl[i - 1] : fminf(ubl[i], u);
                        ubl[0] = fminf(ubl[0], u);
                    }
                } else {
                    // lanes without a query have H32 = -inf; a query with no threshold has
                    // c1f = c2f = 0, H32 = +inf
                    const float L = fmaf(c2f, Ar[r][1], Ar[r][0]);
                    const float Rv = fmaf(c1f, (float)acc, H32);
                    sm[r] = __ballot(L <= Rv);
                }
            }
            if constexpr (!UB_PASS) {
                if ((sm[0] | sm[1] | sm[2] | sm[3]) == 0ull) return;
                // rare: append survivors (sorted position) to the query's list
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if ((sm[r] >> lane) & 1ull) {
                        const int slot = atomicAdd(&a.cand_cnt[q], 1);
                        if (slot < a.cap) a.cand_id[(size_t)q * a.cap + slot] = v0 + li0 + 4 * g + r;
                    }
                }
                if (a.stats) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) st_surv += __popcll(sm[r]);
                }
            }
        };

        // ---- stream the slice through LDS in 64-vector blocks ----
        // A block never crosses a T-tile (T and the block starts are multiples of 64).
        // (The staging values are separate scalars filled by value: an array captured by
        // reference lands in scratch memory and serialises every load.)
        uint4 st0 = make_uint4(0u, 0u, 0u, 0u), st1 = st0, st2 = st0, st3 = st0;
        float2 st_ar = make_float2(0.0f, 0.0f);
        const uint32_t* sq8_c = a.sq8 + (size_t)t0 * D4 * T;  // cluster's first tile
        auto gload = [&](int blk0) {
            const int ct = blk0 / T, cw = blk0 - ct * T;
            const uint32_t* base = sq8_c + (size_t)ct * D4 * T + cw;
            st0 = cell_load(base, 0, tid, D4, T);
            if constexpr (KS > 1) st1 = cell_load(base, 1, tid, D4, T);
            if constexpr (KS > 2) st2 = cell_load(base, 2, tid, D4, T);
            if constexpr (KS > 3) st3 = cell_load(base, 3, tid, D4, T);
            if (tid < kBlkV) {
                const int li = blk0 + tid;
                if (li < ve) {
                    const float2 ar = a.vec_Ar[v0 + li];
                    // lower-bound pass keeps P = A_lo - r^2 (its f32 rounding is inside the
                    // slack), upper-bound pass keeps A_lo
                    st_ar = UB_PASS ? ar : make_float2(fmaf(-ar.y, ar.y, ar.x), ar.y);
                } else {
                    st_ar = make_float2(__int_as_float(0x7fc00000), INFINITY);
                }
            }
        };
        auto lstore = [&](int buf) {
            cell_store(s_codes[buf], st0, 0, tid);
            if constexpr (KS > 1) cell_store(s_codes[buf], st1, 1, tid);
            if constexpr (KS > 2) cell_store(s_codes[buf], st2, 2, tid);
            if constexpr (KS > 3) cell_store(s_codes[buf], st3, 3, tid);
            if (tid < kBlkV) s_ar[buf][tid] = st_ar;
        };
        const int nblk = (ve - vb + kBlkV - 1) / kBlkV;
        if (nblk > 0) gload(vb);
        for (int b = 0; b < nblk; ++b) {
            const int buf = b & 1;
            lstore(buf);
            __syncthreads();
            if (b + 1 < nblk) gload(vb + (b + 1) * kBlkV);
            if (active) {
                const int blk0 = vb + b * kBlkV;
                for (int t = rr; t < kBlkV / 16; t += R) {
                    if (blk0 + t * 16 >= ve) break;
                    tile(buf, t, blk0 + t * 16);
                }
            }
        }
        if (a.stats && active && rr == 0)
            st_cand += (unsigned long long)nq * (unsigned long long)(ve - vb);

        if constexpr (UB_PASS) {
            // K-th smallest upper bound of each query -> atomicMin into tau[q] (float64 bit
            // pattern).  Every lane holds the 16 smallest bounds of its rows.
            //  K <= 16: the four lane groups' lists are merged in registers (exact top 16 of
            //    the wave), replica waves exchange theirs through LDS and the group's first
            //    wave merges them the same way: the K-th entry is the exact K-th smallest.
            //  K > 16: all R x 64 kept values go through a register bitonic list; their K-th
            //    smallest is >= the true K-th smallest bound, so still an upper bound.
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
                    float kth = INFINITY;
#pragma unroll
                    for (int i = 0; i < kUbList; ++i)
                        if (i == a.K - 1) kth = ubl[i];
                    if (kth < INFINITY) {
                        const double u = (double)kth;
                        const double tub = u * u / a.rot_sq_min * (1.0 + 1e-6);
                        atomicMin(reinterpret_cast<unsigned long long*>(a.tau) + q,
                                  (unsigned long long)key_of(tub));
                    }
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
                        uint64_t kk;
                        int32_t ki;
                        L.at(a.K - 1, kk, ki);
                        const int qq = __shfl(q, jj, kWave);
                        if (lane == 0 && dist_of(kk) < (double)INFINITY) {
                            const double u = dist_of(kk);
                            const double tub = u * u / a.rot_sq_min * (1.0 + 1e-6);
                            atomicMin(reinterpret_cast<unsigned long long*>(a.tau) + qq,
                                      (unsigned long long)key_of(tub));
                        }
                    }
                }
            }
        }
    }

    if (a.stats && lane == 0) {
        const int slot = (int)(blockIdx.x % kStatSlots) * 4;
        atomicAdd(&a.stats[slot + 0], st_cand);
        atomicAdd(&a.stats[slot + 1], st_cand * (unsigned long long)D_pad);
        atomicAdd(&a.stats[slot + 2], st_surv);
    }
}

template __global__ void batch_scan_kernel<true, 1>(BatchArgs);
template __global__ void batch_scan_kernel<true, 2>(BatchArgs);
template __global__ void batch_scan_kernel<true, 3>(BatchArgs);
template __global__ void batch_scan_kernel<true, 4>(BatchArgs);
template __global__ void batch_scan_kernel<false, 1>(BatchArgs);
template __global__ void batch_scan_kernel<false, 2>(BatchArgs);
template __global__ void batch_scan_kernel<false, 3>(BatchArgs);
template __global__ void batch_scan_kernel<false, 4>(BatchArgs);

// tau_sq output of the batched route: the seeded float64 threshold, rounded up to float32.
__global__ void tau_to_f32_kernel(const double* tau, float* out, int B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < B) out[i] = __double2float_ru(tau[i]);
}

}  // namespace trident
