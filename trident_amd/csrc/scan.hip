// Per-(cluster, query)-pair scan of the lossless IVF query path on gfx950, plus the
// per-query merge.
//
// One 256-thread workgroup (4 independent waves) per pair; pairs arrive grouped by cluster
// and are remapped so each XCD walks a contiguous run of clusters (its own L2 keeps the
// cluster's codes).  Each wave takes 64-vector slices of the cluster, one vector per lane:
//
//   Stage X (UB)   : upper bound per vector from the SQ8 codes over all dims; the K-th
//                    smallest over the cluster seeds the threshold
//                    (reference src/trident_v4_kernels.cu:626-676).
//   Stage Y        : SQ8 lower bound accumulated block by block; a lane dies once the bound
//                    passes the threshold and the wave leaves the slice as soon as its 64-bit
//                    ballot is empty -- no block barrier (reference :679-780, whose warp32
//                    ballot is followed by a CTA barrier on every block).
//   Stage Z        : survivors are compacted into a per-wave LDS queue with ballot/mbcnt
//                    and refined 64 at a time: the wave copies the survivors' rows into LDS
//                    with coalesced loads, then each lane sums its own row in float64, in
//                    dimension order (the canonical distance) (reference :796-941).
//   top-K          : each wave keeps a register bitonic top-K list; the four lists are
//                    merged at the end and the pair emits at most K entries
//                    (reference :943-961 emission, :19-60 ordering).
//
// The kernel's KIND (enum ScanKind) selects the route:
//   kScanCascade / kScanCascadeUb   mode 2 (Stage Y / Z, with Stage X seeding for the latter);
//   kScanExact                      mode 10, CM-FP32 (reference :268-374): no Stage X/Y, every
//                                   vector refined exactly;
//   kScanTribase                    mode 11, Tribase (reference :379-521): as kScanExact, but a
//                                   vector with | |q - c| - |x - c| | > sqrt(tau) is not refined
//                                   (triangle inequality, margins for the float32 norms);
//   kScanHat                        modes 0 / 1 (reference :529-962, MODE 0 / 1): no refinement;
//                                   vectors are ranked by their SQ8 reconstruction distance in
//                                   the rotated space, acc_hat = sum_d fmaf(code_d, delta_d,
//                                   base_d)^2 in dimension order (base_d = fl32(vmin_d - q_rot,d)),
//                                   keyed (acc_hat bits, original id) with the sorted position as
//                                   the entry's id.
//
// Rigour.  Stage Y prunes x when  lb_f32(x) > round_up(tau * lb_scale)  with
// lb_scale = rot_sq_max * (1 + rho) * (1 + 1e-12), rho = (D_pad + 4) * 2^-24.  Per dimension
// the kernel evaluates a = fma(code, delta, base32) and l = max(|a| - e32, 0), where e32
// (dim_params) bounds eps_dim plus every rounding between the exact rotated gap and a; so
// l <= |x_rot - q_rot| (1 + 2^-24) and the float32 sum exceeds the exact rotated LB by at
// most a factor (1 + rho).  |(x - q) R|^2 <= rot_sq_max |x - q|^2 then gives
// lb_f32 > round_up(tau * lb_scale)  =>  d64(x) > tau.  Stage X mirrors this with
// u = |a| + e32 and ub_scale = (1 + rho) (1 + 1e-12) / rot_sq_min.
#include "common.hpp"
#include "kernels.hpp"

namespace trident {

constexpr int kQueueCap = 128;  // per-wave survivor queue (64 pending + one slice)

__device__ __forceinline__ void dim_params(double vm, float dl, float ep, double xr, double qe,
                                           float& base32, float& e32) {
    const double b64 = vm - xr;
    const float b32 = (float)b64;
    const double E = fabs((double)b32 - b64) + qe + 0x1p-52 * fabs(b64) +
                     0x1p-24 * (255.0 * (double)dl + fabs((double)b32)) * (1.0 + 0x1p-20) +
                     0x1p-126;
    base32 = b32;
    e32 = __double2float_ru(((double)ep + E) * (1.0 + 0x1p-50));
}

__device__ __forceinline__ float lb_step(uint32_t code, float dl, float bs, float ee, float acc) {
    const float a = fmaf((float)code, dl, bs);
    const float l = fmaxf(fabsf(a) - ee, 0.0f);
    return fmaf(l, l, acc);
}

__device__ __forceinline__ float ub_step(uint32_t code, float dl, float bs, float ee, float acc) {
    const float a = fmaf((float)code, dl, bs);
    const float u = fabsf(a) + ee;
    return fmaf(u, u, acc);
}

__device__ __forceinline__ uint32_t tau_bits_of(double tau, double lb_scale) {
    return __float_as_uint(__double2float_ru(tau * lb_scale));
}

template <bool UB>
__device__ __forceinline__ float sq8_accumulate(const uint32_t* cp, int T, int d4s, int d4e,
                                                const float* s_base, const float* s_dlt,
                                                const float* s_e, float acc) {
#pragma unroll 4
    for (int d4 = d4s; d4 < d4e; ++d4) {
        const uint32_t w = cp[(size_t)d4 * T];
        const float4 bs = *reinterpret_cast<const float4*>(s_base + 4 * d4);
        const float4 dl = *reinterpret_cast<const float4*>(s_dlt + 4 * d4);
        const float4 ee = *reinterpret_cast<const float4*>(s_e + 4 * d4);
        if constexpr (UB) {
            acc = ub_step(w & 0xffu, dl.x, bs.x, ee.x, acc);
            acc = ub_step((w >> 8) & 0xffu, dl.y, bs.y, ee.y, acc);
            acc = ub_step((w >> 16) & 0xffu, dl.z, bs.z, ee.z, acc);
            acc = ub_step(w >> 24, dl.w, bs.w, ee.w, acc);
        } else {
            acc = lb_step(w & 0xffu, dl.x, bs.x, ee.x, acc);
            acc = lb_step((w >> 8) & 0xffu, dl.y, bs.y, ee.y, acc);
            acc = lb_step((w >> 16) & 0xffu, dl.z, bs.z, ee.z, acc);
            acc = lb_step(w >> 24, dl.w, bs.w, ee.w, acc);
        }
    }
    return acc;
}

template <int KP>
__device__ __forceinline__ void list_store(const WaveList<KP>& L, uint64_t* k, int32_t* i) {
    const int lane = lane_id();
    k[lane] = L.k0;
    i[lane] = L.i0;
    if constexpr (KP >= 128) {
        k[kWave + lane] = L.k1;
        i[kWave + lane] = L.i1;
    }
    if constexpr (KP == 256) {
        k[2 * kWave + lane] = L.k2;
        i[2 * kWave + lane] = L.i2;
        k[3 * kWave + lane] = L.k3;
        i[3 * kWave + lane] = L.i3;
    }
}

template <int KP>
__device__ __forceinline__ void list_load(WaveList<KP>& L, const uint64_t* k, const int32_t* i) {
    const int lane = lane_id();
    L.k0 = k[lane];
    L.i0 = i[lane];
    if constexpr (KP >= 128) {
        L.k1 = k[kWave + lane];
        L.i1 = i[kWave + lane];
    }
    if constexpr (KP == 256) {
        L.k2 = k[2 * kWave + lane];
        L.i2 = i[2 * kWave + lane];
        L.k3 = k[3 * kWave + lane];
        L.i3 = i[3 * kWave + lane];
    }
}


template <int KP>
__device__ __forceinline__ void list_absorb(WaveList<KP>& L, int K, const uint64_t* k,
                                            const int32_t* i) {
    const int lane = lane_id();
    for_chunks<KP>([&](auto cc) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        if (c * kWave < K) list_offer(L, K, k[c * kWave + lane], i[c * kWave + lane]);
    });
}

__device__ __forceinline__ float hat_step(uint32_t code, float dl, float bs, float acc) {
    const float a = fmaf((float)code, dl, bs);
    return fmaf(a, a, acc);
}

__device__ __forceinline__ float sq8_hat(const uint32_t* cp, int T, int D4, const float* s_base,
                                         const float* s_dlt) {
    float acc = 0.0f;
#pragma unroll 4
    for (int d4 = 0; d4 < D4; ++d4) {
        const uint32_t w = cp[(size_t)d4 * T];
        const float4 bs = *reinterpret_cast<const float4*>(s_base + 4 * d4);
        const float4 dl = *reinterpret_cast<const float4*>(s_dlt + 4 * d4);
        acc = hat_step(w & 0xffu, dl.x, bs.x, acc);
        acc = hat_step((w >> 8) & 0xffu, dl.y, bs.y, acc);
        acc = hat_step((w >> 16) & 0xffu, dl.z, bs.z, acc);
        acc = hat_step(w >> 24, dl.w, bs.w, acc);
    }
    return acc;
}

// Key of a kScanHat entry: ordered by (acc_hat, original id); acc_hat >= 0.
__device__ __forceinline__ uint64_t hat_key(float acc_hat, int32_t oid) {
    return ((uint64_t)__float_as_uint(acc_hat) << 32) | (uint32_t)oid;
}

template <int KP, int KIND>
__global__ __launch_bounds__(256) void pair_scan_kernel(ScanArgs a) {
    constexpr bool CASCADE = KIND == kScanCascade || KIND == kScanCascadeUb;
    constexpr bool UB = KIND == kScanCascadeUb;
    constexpr bool TRI = KIND == kScanTribase;
    constexpr bool HAT = KIND == kScanHat;
    constexpr bool SQ8 = CASCADE || HAT;  // reads the codes
    extern __shared__ __align__(16) unsigned char dyn_smem[];
    __shared__ float s_stage[kWavesPerBlock][kStageCh][kWave + 1];
    __shared__ int32_t s_qspos[kWavesPerBlock][kQueueCap];
    __shared__ int32_t s_qoid[kWavesPerBlock][kQueueCap];
    __shared__ int32_t s_blk[68];
    __shared__ uint32_t s_tau_bits;
    __shared__ double s_thr;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware mapping: consecutive dispatch slots go to different XCDs, so XCD x walks
    // the contiguous pair range [x * nx, (x + 1) * nx) of the cluster-sorted pair list.
    const int nx = (a.M + 7) >> 3;
    const int p = (int)(blockIdx.x & 7) * nx + (int)(blockIdx.x >> 3);
    if (p >= a.M) return;
    const int cid = a.pair_cid[p];
    const int q = a.pair_qid[p];
    const int v0 = a.vec_off[cid];
    const int n = a.vec_off[cid + 1] - v0;
    if (n <= 0) return;
    const int t0 = a.tile_off[cid];
    const int nslices = (n + kWave - 1) / kWave;
    const int D = a.D, D_pad = a.D_pad, T = a.T, K = a.K;
    const int D4 = D_pad >> 2;

    double* s_q64 = reinterpret_cast<double*>(dyn_smem);
    float* s_base = reinterpret_cast<float*>(s_q64 + D);
    float* s_dlt = s_base + D_pad;
    float* s_e = s_dlt + D_pad;

    const double tau_init = a.tau_in ? a.tau_in[q] : (double)INFINITY;
    for (int d = tid; d < D; d += kBlock) s_q64[d] = a.xq64[(size_t)q * D + d];
    if constexpr (SQ8) {
        const size_t off = a.per_cluster ? (size_t)cid * D_pad : 0;
        const double* xr = a.xrot64 + (size_t)q * D_pad;
        const double* qe = a.qerr + (size_t)q * D_pad;
        for (int d = tid; d < D_pad; d += kBlock) {
            float b32, e32;
            dim_params((double)a.vmin[off + d], a.delta[off + d], a.eps[off + d], xr[d], qe[d],
                       b32, e32);
            s_base[d] = b32;
            s_dlt[d] = a.delta[off + d];
            s_e[d] = e32;
        }
        for (int b = tid; b <= a.nb; b += kBlock) s_blk[b] = a.blk[b];
    }
    if (tid == 0) {
        s_thr = tau_init;
        s_tau_bits = tau_bits_of(tau_init, a.lb_scale);
    }
    __syncthreads();

    const uint32_t* sq8c = a.sq8 + (size_t)t0 * D4 * T;
    uint64_t* s_ck = reinterpret_cast<uint64_t*>(&s_stage[0][0][0]);
    int32_t* s_ci = reinterpret_cast<int32_t*>(s_ck + kWavesPerBlock * KP);

    // ---------------- Stage X: SQ8 upper-bound threshold seeding ----------------
    if constexpr (CASCADE && UB) {
        WaveList<KP> U;
        U.init();
        for (int s = wid; s < nslices; s += kWavesPerBlock) {
            const int li = s * kWave + lane;
            const bool valid = li < n;
            const uint32_t* cp = sq8c + (size_t)(s / (T / kWave)) * D4 * T +
                                 (s % (T / kWave)) * kWave + lane;
            float ub = 0.0f;
            if (valid) ub = sq8_accumulate<true>(cp, T, 0, D4, s_base, s_dlt, s_e, 0.0f);
            list_offer(U, K, valid ? key_of((double)ub) : kKeyInvalid, valid ? li : kIdInvalid);
        }
        list_store(U, s_ck + wid * KP, s_ci + wid * KP);
        __syncthreads();
        if (wid == 0) {
            for (int w = 1; w < kWavesPerBlock; ++w) list_absorb(U, K, s_ck + w * KP, s_ci + w * KP);
            uint64_t kk;
            int32_t ki;
            U.at(K - 1, kk, ki);
            if (kk != kKeyInvalid && lane == 0) {
                const double tub = dist_of(kk) * a.ub_scale;
                if (tub < s_thr) {
                    s_thr = tub;
                    s_tau_bits = tau_bits_of(tub, a.lb_scale);
                }
            }
        }
        __syncthreads();
    }

    // ---------------- Stage Y / Z ----------------
    WaveList<KP> L;
    L.init();
    double thr = s_thr;
    int qn = 0;
    unsigned long long st_cand = 0, st_dims = 0, st_surv = 0, st_ins = 0;
    int32_t* my_qspos = s_qspos[wid];
    int32_t* my_qoid = s_qoid[wid];
    float(*my_stage)[kWave + 1] = s_stage[wid];

    auto flush = [&](int cnt) {
        const double d64 = refine_rows(a.xb, nullptr, D, my_qspos, cnt, my_stage, s_q64);
        if (a.host_rows && lane == 0) atomicAdd(a.host_rows, (unsigned long long)cnt);
        const bool ok = lane < cnt && d64 <= thr;
        if (a.stats) st_ins += __popcll(__ballot(ok));
        if (list_offer(L, K, ok ? key_of(d64) : kKeyInvalid, ok ? my_qoid[lane] : kIdInvalid)) {
            uint64_t kk;
            int32_t ki;
            L.at(K - 1, kk, ki);
            if (kk != kKeyInvalid) {
                const double kth = dist_of(kk);
                if (kth < thr) {
                    thr = kth;
                    if (CASCADE && lane == 0) atomicMin(&s_tau_bits, tau_bits_of(kth, a.lb_scale));
                }
            }
        }
    };

    for (int s = wid; s < nslices; s += kWavesPerBlock) {
        const int li = s * kWave + lane;
        const bool valid = li < n;
        bool alive = valid;
        if constexpr (HAT) {
            // no refinement: the lane's vector enters the wave list by its reconstruction distance
            const int tile = s / (T / kWave), sub = s % (T / kWave);
            const uint32_t* cp = sq8c + (size_t)tile * D4 * T + sub * kWave + lane;
            const float hat = valid ? sq8_hat(cp, T, D4, s_base, s_dlt) : 0.0f;
            const int32_t oid = valid ? a.tile_oids[(size_t)t0 * T + li] : 0;
            if (a.stats) {
                const int nv = __popcll(__ballot(valid));
                st_cand += nv;
                st_dims += (unsigned long long)nv * (unsigned)D_pad;
            }
            list_offer(L, K, valid ? hat_key(hat, oid) : kKeyInvalid, valid ? v0 + li : kIdInvalid);
            continue;
        }
        if constexpr (TRI) {
            // Tribase: |q - x| >= | |q - c| - |x - c| |.  Both norms are float32 values within
            // 1e-5 (relative) of the exact ones (|q - c| is the rounded float64 norm, |x - c| the
            // index's r_vec_sorted); thr is this wave's running K-th distance, so a skipped
            // vector has d64 > thr and cannot enter the top K.
            if (a.stats) st_cand += __popcll(__ballot(valid));
            if (valid && thr < (double)INFINITY) {
                const double dqc = (double)a.pair_dqc[p], rx = (double)a.r_vec[v0 + li];
                const double tol = 1e-5 * (dqc + rx) + 1e-30;
                if (fabs(dqc - rx) - tol > sqrt(thr) * (1.0 + 1e-6)) alive = false;
            }
            if (a.stats) {
                const int na = __popcll(__ballot(alive));
                st_dims += (unsigned long long)na * (unsigned)D;
                st_surv += na;
            }
        }
        if constexpr (CASCADE) {
            const int tile = s / (T / kWave), sub = s % (T / kWave);
            const float tau_s = __uint_as_float(__atomic_load_n(&s_tau_bits, __ATOMIC_RELAXED));
            if (a.use_l1 && a.tile_rmm && a.pair_dqc) {
                // Residual-norm band |d_qc - |x - c|| <= |q - x| (reference :686-695), with
                // margins for the float32 storage of both norms.
                const double tq = (double)__uint_as_float(
                    __atomic_load_n(&s_tau_bits, __ATOMIC_RELAXED));
                if (tq < (double)INFINITY) {
                    const double dqc = (double)a.pair_dqc[p];
                    const double rmin = (double)a.tile_rmm[(size_t)(t0 + tile) * 2];
                    const double rmax = (double)a.tile_rmm[(size_t)(t0 + tile) * 2 + 1];
                    const double tol = sqrt(tq) * (1.0 + 1e-6) + 1e-6 * (dqc + rmax) + 1e-30;
                    if (rmax + tol < dqc || rmin - tol > dqc) alive = false;
                }
            }
            const uint32_t* cp = sq8c + (size_t)tile * D4 * T + sub * kWave + lane;
            float acc = 0.0f;
            if (a.stats) st_cand += __popcll(__ballot(valid));
            for (int b = 0; b < a.nb; ++b) {
                const uint64_t m = __ballot(alive);
                if (m == 0) break;
                const int d4s = s_blk[b], d4e = s_blk[b + 1];
                if (a.stats) st_dims += (unsigned long long)__popcll(m) * (unsigned)(4 * (d4e - d4s));
                if (alive) {
                    acc = sq8_accumulate<false>(cp, T, d4s, d4e, s_base, s_dlt, s_e, acc);
                    alive = acc <= tau_s;
                }
            }
        }
        const uint64_t m = __ballot(alive);
        const int cnt = __popcll(m);
        if (CASCADE && a.stats) st_surv += (unsigned long long)cnt;
        if (alive) {
            const int pos = qn + mask_rank(m);
            my_qspos[pos] = v0 + li;
            my_qoid[pos] = a.tile_oids[(size_t)t0 * T + li];
        }
        qn += cnt;
        if (qn >= kWave) {
            wave_sync();
            flush(kWave);
            const int rest = qn - kWave;
            int32_t sp = 0, oi = 0;
            if (lane < rest) {
                sp = my_qspos[kWave + lane];
                oi = my_qoid[kWave + lane];
            }
            wave_sync();
            if (lane < rest) {
                my_qspos[lane] = sp;
                my_qoid[lane] = oi;
            }
            qn = rest;
            wave_sync();
        }
    }
    if (qn > 0) {
        wave_sync();
        flush(qn);
    }
    // ---------------- combine the four wave lists and emit <= K entries ----------------
    __syncthreads();
    list_store(L, s_ck + wid * KP, s_ci + wid * KP);
    if (a.stats) {
        // Telemetry: one atomic per counter per workgroup, spread over kStatSlots slots that
        // stats_fold_kernel sums afterwards (a single address would serialise every workgroup).
        unsigned long long* s_st = reinterpret_cast<unsigned long long*>(s_ci + kWavesPerBlock * KP);
        if (lane == 0) {
            s_st[wid * 4 + 0] = st_cand;
            s_st[wid * 4 + 1] = st_dims;
            s_st[wid * 4 + 2] = st_surv;
            s_st[wid * 4 + 3] = st_ins;
        }
        __syncthreads();
        if (tid < 4) {
            unsigned long long v = 0;
            for (int w = 0; w < kWavesPerBlock; ++w) v += s_st[w * 4 + tid];
            if (v) atomicAdd(&a.stats[(blockIdx.x % kStatSlots) * 4 + tid], v);
        }
    }
    __syncthreads();
    if (wid != 0) return;
    for (int w = 1; w < kWavesPerBlock; ++w) list_absorb(L, K, s_ck + w * KP, s_ci + w * KP);
    // valid entries are a prefix of the sorted list
    int cnt = 0;
    for_chunks<KP>([&](auto cc) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        uint64_t k;
        int32_t i;
        list_chunk<c>(L, k, i);
        cnt += __popcll(__ballot(c * kWave + lane < K && k != kKeyInvalid));
    });
    if (cnt == 0) return;
    int base = 0;
    if (lane == 0) base = atomicAdd(&a.cand_cnt[q], cnt);
    base = __builtin_amdgcn_readfirstlane(base);
    if (base + cnt > a.cap) return;  // unreachable: cap >= nprobe * K
    uint64_t* ck = a.cand_key + (size_t)q * a.cap + base;
    int32_t* ci = a.cand_id + (size_t)q * a.cap + base;
    for_chunks<KP>([&](auto cc) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        uint64_t k;
        int32_t i;
        list_chunk<c>(L, k, i);
        if (c * kWave + lane < cnt) {
            ck[c * kWave + lane] = k;
            ci[c * kWave + lane] = i;
        }
    });
}

// Sums the kStatSlots telemetry slots into the caller's int64[4] (added to its contents).
__global__ void stats_fold_kernel(const unsigned long long* slots, int64_t* out) {
    const int k = threadIdx.x;
    if (k >= 4) return;
    unsigned long long v = 0;
    for (int s = 0; s < kStatSlots; ++s) v += slots[s * 4 + k];
    out[k] += (int64_t)v;
}

// One wave per query: merges the pass's candidates (and the previous pass's list) into
// the query's top list; writes the K-th distance and, on the final pass, the outputs.
// Bounded rescan of an overflowed list (one wave, query q): pass UB = true offers every probed
// row's Stage X upper bound (mapped to the float64 distance, as the per-pair scan) to L, so
// that L's K-th entry bounds the K-th distance; pass UB = false reads and refines exactly only
// the rows whose Stage Y lower bound does not exceed round_up(t * lb_scale) -- every row of the
// exact top-K, since lb <= d64 <= t for them.  The per-dim constants of each (q, cluster) pair
// are staged in the wave's LDS (3 D_pad floats); codes come from the batched route's cells
// (c ^ 0x80, 16 dims a cell).
// One probed cluster (probe p of query q) of an overflowed list's rescan: UB offers every row's
// SQ8 upper bound (key, sorted position) to L; otherwise the rows whose lower bound is within t
// are refined (canonical float64 distance) and offered as (distance, original id).  s_par holds
// 3 D_pad floats of the wave's LDS.
template <int KP, bool UB>
__device__ __forceinline__ void ovf_cluster_pass(const MergeArgs& a, int q, int p, WaveList<KP>& L,
                                                 double t, float* s_par) {
    const int lane = lane_id();
    const int D_pad = a.D_pad, T = a.T, G16 = D_pad >> 4;
    const int V = D_pad <= 256 ? 64 : 16;
    float *s_bs = s_par, *s_dl = s_par + D_pad, *s_e = s_par + 2 * D_pad;
    const double* qv = a.xq64 + (size_t)q * a.D;
    const uint32_t tb = UB ? 0u : tau_bits_of(t, a.lb_scale);
    {
        const int c = a.probe_cids[(size_t)q * a.nprobe + p];
        const int v0 = a.vec_off[c], n = a.vec_off[c + 1] - v0, t0 = a.tile_off[c];
        const size_t off = a.per_cluster ? (size_t)c * D_pad : 0;
        wave_sync();  // the previous cluster's constants are no longer read
        for (int d = lane; d < D_pad; d += kWave) {
            float b32, e32;
            dim_params((double)a.vmin[off + d], a.delta[off + d], a.eps[off + d],
                       a.xrot64[(size_t)q * D_pad + d], a.qerr[(size_t)q * D_pad + d], b32, e32);
            s_bs[d] = b32;
            s_dl[d] = a.delta[off + d];
            s_e[d] = e32;
        }
        wave_sync();
        for (int b0 = 0; b0 < n; b0 += kWave) {
            const int l = b0 + lane;
            const bool in = l < n;
            const int tile = t0 + (in ? l : 0) / T, slot = (in ? l : 0) % T;
            float acc = 0.0f;
            if (in) {
                for (int g = 0; g < G16; ++g) {
                    const uint4 cw = a.cells[((size_t)(tile * (T / V) + slot / V) * G16 + g) * V + slot % V];
                    const uint32_t w[4] = {cw.x ^ 0x80808080u, cw.y ^ 0x80808080u,
                                           cw.z ^ 0x80808080u, cw.w ^ 0x80808080u};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
#pragma unroll
                        for (int by = 0; by < 4; ++by) {
                            const int d = 16 * g + 4 * k + by;
                            const uint32_t cd = (w[k] >> (8 * by)) & 0xffu;
                            acc = UB ? ub_step(cd, s_dl[d], s_bs[d], s_e[d], acc)
                                     : lb_step(cd, s_dl[d], s_bs[d], s_e[d], acc);
                        }
                }
            }
            if constexpr (UB) {
                list_offer(L, a.K, in ? key_of((double)acc * a.ub_scale) : kKeyInvalid,
                           in ? v0 + l : kIdInvalid);
            } else {
                const bool need = in && __float_as_uint(acc) <= tb;
                if (a.host_rows && lane == 0)
                    atomicAdd(a.host_rows, (unsigned long long)__popcll(__ballot(need)));
                uint64_t k = kKeyInvalid;
                int32_t id = kIdInvalid;
                if (need) {
                    const float* xr = a.xb + (size_t)(v0 + l) * a.D;
                    double d64 = 0.0;
                    for (int d = 0; d < a.D; ++d) {
                        const double tt = (double)xr[d] - qv[d];
                        d64 = fma(tt, tt, d64);
                    }
                    k = key_of(d64);
                    id = a.tile_oids[(size_t)tile * T + slot];
                }
                list_offer(L, a.K, k, id);
            }
        }
    }
}

template <int KP, bool UB>
__device__ __forceinline__ void ovf_bounded_pass(const MergeArgs& a, int q, WaveList<KP>& L, double t,
                                              float* s_par) {
    for (int p = 0; p < a.nprobe; ++p) ovf_cluster_pass<KP, UB>(a, q, p, L, t, s_par);
}

// Parallel form of the bounded rescan.  An overflowed query's slot holds, per probe, the K best
// entries of that probe's cluster: every member of the query's top-K over all probed rows is
// among its own cluster's K best, so merging the per-probe lists gives the same result as one
// list over every probed row (the serial rescan).
__global__ void ovf_collect_kernel(MergeArgs a) {
    const int q = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (q >= a.B) return;
    int slot = -1;
    if (a.cand_cnt[q] > a.cap) {
        const int s = atomicAdd(a.ovf_n, 1);
        if (s < a.ovf_max) {
            slot = s;
            a.ovf_q[s] = q;
        }
    }
    a.ovf_slot[q] = slot;
}

// One wave per (slot, probe) item, grid-strided (the grid is sized for the slots, items past the
// taken slots end the loop at once): UB lists the cluster's K smallest upper bounds, else its K
// best refined rows among those whose lower bound is within the slot's threshold.
template <int KP, bool UB>
__global__ __launch_bounds__(256) void ovf_scan_kernel(MergeArgs a) {
    extern __shared__ float s_ovf[];  // 3 D_pad floats per wave
    const int wid = (int)(threadIdx.x >> 6);
    const int n = __builtin_amdgcn_readfirstlane(min(*a.ovf_n, a.ovf_max)) * a.nprobe;
    float* s_par = s_ovf + wid * 3 * a.D_pad;
    for (int it = (int)blockIdx.x * kWavesPerBlock + wid; it < n; it += (int)gridDim.x * kWavesPerBlock) {
        const int slot = it / a.nprobe, p = it - slot * a.nprobe;
        const int q = a.ovf_q[slot];
        WaveList<KP> L;
        L.init();
        ovf_cluster_pass<KP, UB>(a, q, p, L, UB ? 0.0 : a.ovf_t[slot], s_par);
        list_store(L, a.ovf_key + (size_t)it * KP, a.ovf_id + (size_t)it * KP);
    }
}

// One wave per taken slot: the K-th smallest upper bound over the slot's per-probe lists (and
// the pass's threshold) bounds the query's K-th distance.
template <int KP>
__global__ __launch_bounds__(256) void ovf_kth_kernel(MergeArgs a) {
    const int lane = threadIdx.x & 63;
    const int slot = (int)blockIdx.x * kWavesPerBlock + (int)(threadIdx.x >> 6);
    if (slot >= min(*a.ovf_n, a.ovf_max)) return;
    const int q = a.ovf_q[slot];
    const int total = a.nprobe * KP;
    const uint64_t* k = a.ovf_key + (size_t)slot * total;
    const int32_t* id = a.ovf_id + (size_t)slot * total;
    WaveList<KP> L;
    L.init();
    for (int e0 = 0; e0 < total; e0 += kWave) {
        const int e = e0 + lane;
        list_offer(L, a.K, e < total ? k[e] : kKeyInvalid, e < total ? id[e] : kIdInvalid);
    }
    uint64_t kk;
    int32_t ki;
    L.at(a.K - 1, kk, ki);
    if (lane == 0) a.ovf_t[slot] = fmin(a.tau64[q], kk != kKeyInvalid ? dist_of(kk) : (double)INFINITY);
}

template <int KP>
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
    extern __shared__ float s_ovf[];  // ovf_bounds: 3 D_pad floats per wave
    const int lane = threadIdx.x & 63;
    const int q = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (q >= a.B) return;
    WaveList<KP> L;
    L.init();
    uint64_t* lk = a.list_key + (size_t)q * KP;
    int32_t* li = a.list_id + (size_t)q * KP;
    if (a.use_prev) list_load(L, lk, li);
    const int raw = a.cand_cnt[q];
    const int oslot = raw > a.cap && a.ovf_par ? a.ovf_slot[q] : -1;
    if (oslot >= 0) {
        // Overflowed list rescanned in parallel (ovf_scan_kernel): merge its per-probe lists.
        L.init();
        const int total = a.nprobe * KP;
        const uint64_t* k = a.ovf_key + (size_t)oslot * total;
        const int32_t* id = a.ovf_id + (size_t)oslot * total;
        for (int e0 = 0; e0 < total; e0 += kWave) {
            const int e = e0 + lane;
            list_offer(L, a.K, e < total ? k[e] : kKeyInvalid, e < total ? id[e] : kIdInvalid);
        }
    } else if (raw > a.cap && a.probe_cids && a.ovf_bounds) {
        // Overflowed list, SQ8 codes at hand: the K-th smallest upper bound over the probed rows
        // (and the pass's threshold) bounds the K-th distance; only rows whose lower bound
        // passes it are read and refined.
        float* s_par = s_ovf + (threadIdx.x >> 6) * 3 * a.D_pad;
        L.init();
        ovf_bounded_pass<KP, true>(a, q, L, 0.0, s_par);
        uint64_t kk;
        int32_t ki;
        L.at(a.K - 1, kk, ki);
        const double t = fmin(a.tau64[q], kk != kKeyInvalid ? dist_of(kk) : (double)INFINITY);
        L.init();
        ovf_bounded_pass<KP, false>(a, q, L, t, s_par);
    } else if (raw > a.cap && a.probe_cids) {
        // Overflowed list: rescan every probed vector exactly (canonical float64 distance).
        L.init();
        const double* qv = a.xq64 + (size_t)q * a.D;
        for (int p = 0; p < a.nprobe; ++p) {
            const int c = a.probe_cids[(size_t)q * a.nprobe + p];
            const int v0 = a.vec_off[c], n = a.vec_off[c + 1] - v0, t0 = a.tile_off[c];
            if (a.host_rows && lane == 0) atomicAdd(a.host_rows, (unsigned long long)max(n, 0));
            for (int b0 = 0; b0 < n; b0 += kWave) {
                const int li = b0 + lane;
                uint64_t k = kKeyInvalid;
                int32_t id = kIdInvalid;
                if (li < n) {
                    const float* xr = a.xb + (size_t)(v0 + li) * a.D;
                    double acc = 0.0;
                    for (int d = 0; d < a.D; ++d) {
                        const double t = (double)xr[d] - qv[d];
                        acc = fma(t, t, acc);
                    }
                    k = key_of(acc);
                    id = a.tile_oids[(size_t)t0 * a.T + li];
                }
                list_offer(L, a.K, k, id);
            }
        }
    } else {
        const int cnt = min(raw, a.cap);
        const uint64_t* ck = a.cand_key + (size_t)q * a.cap;
        const int32_t* ci = a.cand_id + (size_t)q * a.cap;
        for (int b0 = 0; b0 < cnt; b0 += kWave) {
            const int i = b0 + lane;
            list_offer(L, a.K, i < cnt ? ck[i] : kKeyInvalid, i < cnt ? ci[i] : kIdInvalid);
        }
    }
    list_store(L, lk, li);
    uint64_t kk;
    int32_t ki;
    L.at(a.K - 1, kk, ki);
    const bool full = kk != kKeyInvalid;
    if (lane == 0) {
        if (a.hat) {
            // acc_hat orders the list but bounds no exact distance
            a.tau64[q] = (double)INFINITY;
            if (a.tau_sq_out) a.tau_sq_out[q] = full ? __uint_as_float((uint32_t)(kk >> 32)) : INFINITY;
        } else {
            a.tau64[q] = full ? dist_of(kk) : (double)INFINITY;
            if (a.tau_sq_out) a.tau_sq_out[q] = full ? __double2float_ru(dist_of(kk)) : INFINITY;
        }
    }
    if (a.out_d) {
        float* od = a.out_d + (size_t)q * a.K;
        int64_t* oi = a.out_i + (size_t)q * a.K;
        for_chunks<KP>([&](auto cc) __attribute__((always_inline)) {
            constexpr int c = decltype(cc)::value;
            uint64_t k;
            int32_t i;
            list_chunk<c>(L, k, i);
            const int r = c * kWave + lane;
            if (r < a.K) {
                const bool v = k != kKeyInvalid;
                if (a.hat) {
                    od[r] = v ? __uint_as_float((uint32_t)(k >> 32)) : INFINITY;
                    oi[r] = v ? (int64_t)(int32_t)(uint32_t)k : -1;
                } else {
                    od[r] = v ? (float)dist_of(k) : INFINITY;
                    oi[r] = v ? (int64_t)i : -1;
                }
            }
        });
    }
}

// Mode 0's exact rerank of the merged top-M list (RerankArgs).  Wave w refines list entries
// 64 w .. 64 w + 63 with the per-pair scan's staged float64 rows (refine_rows), keys them
// (distance, original id) and the workgroup keeps the K <= KO best.
template <int KO>
__global__ __launch_bounds__(256) void rerank_kernel(RerankArgs a) {
    extern __shared__ __align__(16) unsigned char dyn_smem[];
    __shared__ float s_stage[kWavesPerBlock][kStageCh][kWave + 1];
    __shared__ int32_t s_spos[kWavesPerBlock][kWave];
    __shared__ uint64_t s_ok[kWavesPerBlock][KO];
    __shared__ int32_t s_oi[kWavesPerBlock][KO];
    const int q = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    double* s_q64 = reinterpret_cast<double*>(dyn_smem);
    for (int d = tid; d < a.D; d += kBlock) s_q64[d] = a.xq64[(size_t)q * a.D + d];
    __syncthreads();
    const int r = wid * kWave + lane;
    const bool in = r < a.M && r < a.KP;
    const uint64_t hk = in ? a.list_key[(size_t)q * a.KP + r] : kKeyInvalid;
    const bool v = hk != kKeyInvalid;
    const int32_t spos = v ? a.list_id[(size_t)q * a.KP + r] : 0;
    // valid entries are a prefix of the sorted list, so each wave's are a prefix of its 64
    const int nv = __popcll(__ballot(v));
    s_spos[wid][lane] = spos;
    wave_sync();
    double d64 = 0.0;
    if (nv > 0) d64 = refine_rows(a.xb, nullptr, a.D, s_spos[wid], nv, s_stage[wid], s_q64);
    if (a.host_rows && lane == 0 && nv > 0) atomicAdd(a.host_rows, (unsigned long long)nv);
    WaveList<KO> L;
    L.init();
    list_offer(L, a.K, v ? key_of(d64) : kKeyInvalid, v ? (int32_t)(uint32_t)hk : kIdInvalid);
    list_store(L, s_ok[wid], s_oi[wid]);
    __syncthreads();
    if (wid != 0) return;
    for (int w = 1; w < kWavesPerBlock; ++w) list_absorb(L, a.K, s_ok[w], s_oi[w]);
    float* od = a.out_d + (size_t)q * a.K;
    int64_t* oi = a.out_i + (size_t)q * a.K;
    for_chunks<KO>([&](auto cc) __attribute__((always_inline)) {
        constexpr int c = decltype(cc)::value;
        uint64_t k;
        int32_t i;
        list_chunk<c>(L, k, i);
        const int rr = c * kWave + lane;
        if (rr < a.K) {
            const bool ok = k != kKeyInvalid;
            od[rr] = ok ? (float)dist_of(k) : INFINITY;
            oi[rr] = ok ? (int64_t)i : -1;
        }
    });
}

// One thread per (query, sorted position) pair: the Stage Y lower bound and the Stage X
// upper bound over all dims, evaluated with exactly the scan kernel's arithmetic, then mapped
// to bounds on the canonical float64 distance: lb = lb_f32 / lb_scale, ub = ub_f32 * ub_scale.
__global__ void sq8_bounds_kernel(ScanArgs a, const int32_t* __restrict__ qids,
                                  const int32_t* __restrict__ cids,
                                  const int64_t* __restrict__ spos, int n, double* lb,
                                  double* ub) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int q = qids[i], cid = cids[i];
    const int li = (int)(spos[i] - a.vec_off[cid]);
    const int s = li / kWave, l = li % kWave;
    const int D_pad = a.D_pad, T = a.T, D4 = D_pad >> 2;
    const int tile = a.tile_off[cid] + s / (T / kWave), sub = s % (T / kWave);
    const uint32_t* cp = a.sq8 + (size_t)tile * D4 * T + sub * kWave + l;
    const size_t off = a.per_cluster ? (size_t)cid * D_pad : 0;
    float acc_l = 0.0f, acc_u = 0.0f;
    for (int d4 = 0; d4 < D4; ++d4) {
        const uint32_t w = cp[(size_t)d4 * T];
        for (int j = 0; j < 4; ++j) {
            const int d = 4 * d4 + j;
            float b32, e32;
            dim_params((double)a.vmin[off + d], a.delta[off + d], a.eps[off + d],
                       a.xrot64[(size_t)q * D_pad + d], a.qerr[(size_t)q * D_pad + d], b32, e32);
            const uint32_t c = (w >> (8 * j)) & 0xffu;
            acc_l = lb_step(c, a.delta[off + d], b32, e32, acc_l);
            acc_u = ub_step(c, a.delta[off + d], b32, e32, acc_u);
        }
    }
    lb[i] = (double)acc_l / a.lb_scale;
    ub[i] = (double)acc_u * a.ub_scale;
}

template __global__ void pair_scan_kernel<64, kScanCascade>(ScanArgs);
template __global__ void pair_scan_kernel<64, kScanCascadeUb>(ScanArgs);
template __global__ void pair_scan_kernel<64, kScanExact>(ScanArgs);
template __global__ void pair_scan_kernel<64, kScanTribase>(ScanArgs);
template __global__ void pair_scan_kernel<64, kScanHat>(ScanArgs);
template __global__ void pair_scan_kernel<128, kScanCascade>(ScanArgs);
template __global__ void pair_scan_kernel<128, kScanCascadeUb>(ScanArgs);
template __global__ void pair_scan_kernel<128, kScanExact>(ScanArgs);
template __global__ void pair_scan_kernel<128, kScanTribase>(ScanArgs);
template __global__ void pair_scan_kernel<128, kScanHat>(ScanArgs);
template __global__ void pair_scan_kernel<256, kScanHat>(ScanArgs);
template __global__ void ovf_scan_kernel<64, true>(MergeArgs);
template __global__ void ovf_scan_kernel<64, false>(MergeArgs);
template __global__ void ovf_scan_kernel<128, true>(MergeArgs);
template __global__ void ovf_scan_kernel<128, false>(MergeArgs);
template __global__ void ovf_kth_kernel<64>(MergeArgs);
template __global__ void ovf_kth_kernel<128>(MergeArgs);
template __global__ void merge_kernel<64>(MergeArgs);
template __global__ void merge_kernel<128>(MergeArgs);
template __global__ void merge_kernel<256>(MergeArgs);
template __global__ void rerank_kernel<64>(RerankArgs);
template __global__ void rerank_kernel<128>(RerankArgs);

}  // namespace trident
