// Device helpers shared by the gfx950 kernels of the lossless IVF query path.
//
// Ordering contract: candidates are ordered lexicographically by (distance, id), the
// tie-break of insert_topk (reference src/trident_v4_kernels.cu:19-60).  Distances are
// non-negative float64 values, so their IEEE bit patterns order like the values and a
// candidate is a (uint64 key, int32 id) pair.  Empty slots hold (kKeyInvalid, kIdInvalid)
// and sort after every real candidate (NaN distances sort after +inf).
//
// Top-K lists live in registers of one wave64: a 64-entry list is one entry per lane, a
// 128- (256-) entry list two (four) entries per lane, sorted ascending across lanes.  Inserting a
// batch of up to 64 candidates is a register bitonic sort of the batch followed by a
// bitonic merge with the list -- no LDS, no block barrier, no single-lane insertion loop.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace trident {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr uint64_t kKeyInvalid = ~0ull;
constexpr int32_t kIdInvalid = 0x7fffffff;

__device__ __forceinline__ uint64_t key_of(double d) {
    return (uint64_t)__double_as_longlong(d);
}
__device__ __forceinline__ double dist_of(uint64_t k) {
    return __longlong_as_double((long long)k);
}
__device__ __forceinline__ bool ent_less(uint64_t ka, int32_t ia, uint64_t kb, int32_t ib) {
    return ka < kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// Index of this lane among the set lanes of `mask` below it.
__device__ __forceinline__ int mask_rank(uint64_t mask) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    int lo = __shfl_xor((int)(uint32_t)v, m, kWave);
    int hi = __shfl_xor((int)(uint32_t)(v >> 32), m, kWave);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Lane src's value of v (ds_bpermute twice).
__device__ __forceinline__ double shfl_f64(double v, int src) {
    const uint64_t k = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)k, src, kWave);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(k >> 32), src, kWave);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

// Block-wide exclusive scan of one uint32 per thread (blocks of kBlock threads); *total (when
// given) receives the block's sum.  Two barriers: s_wave_tot may be reused right after.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave_tot,
                                                         uint32_t* total) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = (uint32_t)__shfl_up((int)inc, o, kWave);
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

// Orders this wave's LDS accesses around the call (producer/consumer inside one wave).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Compare-exchange with lane ^ j; keep the smaller entry when take_min.
__device__ __forceinline__ void cmpx(uint64_t& k, int32_t& id, int j, bool take_min) {
    uint64_t pk = shfl_xor_u64(k, j);
    int32_t pi = __shfl_xor(id, j, kWave);
    bool sw = take_min ? ent_less(pk, pi, k, id) : ent_less(k, id, pk, pi);
    k = sw ? pk : k;
    id = sw ? pi : id;
}

// Full bitonic sort of one entry per lane, ascending across lanes.
__device__ __forceinline__ void wave_sort64(uint64_t& k, int32_t& id) {
    const int lane = lane_id();
#pragma unroll
    for (int s = 2; s <= kWave; s <<= 1) {
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1) {
            const bool up = (lane & s) == 0;
            const bool lower = (lane & j) == 0;
            cmpx(k, id, j, lower == up);
        }
    }
}

// Sorts a bitonic sequence held one entry per lane, ascending.
__device__ __forceinline__ void wave_merge64(uint64_t& k, int32_t& id) {
    const int lane = lane_id();
#pragma unroll
    for (int j = kWave >> 1; j > 0; j >>= 1) cmpx(k, id, j, (lane & j) == 0);
}

template <int KP>
struct WaveList;

// Best 64 candidates seen, one per lane, sorted ascending.
template <>
struct WaveList<64> {
    uint64_t k0;
    int32_t i0;
    __device__ __forceinline__ void init() {
        k0 = kKeyInvalid;
        i0 = kIdInvalid;
    }
    __device__ __forceinline__ void at(int idx, uint64_t& k, int32_t& i) const {
        k = readlane_u64(k0, idx);
        i = __builtin_amdgcn_readlane(i0, idx);
    }
    // Merge an unsorted batch (one entry per lane) into the list.
    __device__ __forceinline__ void insert(uint64_t bk, int32_t bi) {
        wave_sort64(bk, bi);
        uint64_t rk = shfl_xor_u64(bk, kWave - 1);  // lane i <- batch[63 - i]
        int32_t ri = __shfl_xor(bi, kWave - 1, kWave);
        if (ent_less(rk, ri, k0, i0)) {
            k0 = rk;
            i0 = ri;
        }
        wave_merge64(k0, i0);
    }
};

// Best 128 candidates seen: k0/i0 hold ranks 0..63, k1/i1 ranks 64..127.
template <>
struct WaveList<128> {
    uint64_t k0, k1;
    int32_t i0, i1;
    __device__ __forceinline__ void init() {
        k0 = k1 = kKeyInvalid;
        i0 = i1 = kIdInvalid;
    }
    __device__ __forceinline__ void at(int idx, uint64_t& k, int32_t& i) const {
        if (idx < kWave) {
            k = readlane_u64(k0, idx);
            i = __builtin_amdgcn_readlane(i0, idx);
        } else {
            k = readlane_u64(k1, idx - kWave);
            i = __builtin_amdgcn_readlane(i1, idx - kWave);
        }
    }
    __device__ __forceinline__ void insert(uint64_t bk, int32_t bi) {
        wave_sort64(bk, bi);
        uint64_t rk = shfl_xor_u64(bk, kWave - 1);
        int32_t ri = __shfl_xor(bi, kWave - 1, kWave);
        // Ranks 0..63 of the list always survive a 64-entry batch; the other 64 survivors are
        // the smallest 64 of (upper half U, batch): min(U[i], batch[63-i]) is bitonic.
        if (ent_less(rk, ri, k1, i1)) {
            k1 = rk;
            i1 = ri;
        }
        wave_merge64(k1, i1);
        // Bitonic merge of (lower half, reversed new upper half), 128 entries.
        uint64_t mk = shfl_xor_u64(k1, kWave - 1);
        int32_t mi = __shfl_xor(i1, kWave - 1, kWave);
        const bool m_lo = ent_less(mk, mi, k0, i0);
        uint64_t lo_k = m_lo ? mk : k0, hi_k = m_lo ? k0 : mk;
        int32_t lo_i = m_lo ? mi : i0, hi_i = m_lo ? i0 : mi;
        wave_merge64(lo_k, lo_i);
        wave_merge64(hi_k, hi_i);
        k0 = lo_k;
        i0 = lo_i;
        k1 = hi_k;
        i1 = hi_i;
    }
};

// Two sorted 64-entry sequences (a, b) -> the 64 smallest (a) and 64 largest (b) of their union,
// each sorted: min / max of a[i] and b[63 - i] are bitonic.
__device__ __forceinline__ void merge_halves(uint64_t& ak, int32_t& ai, uint64_t& bk, int32_t& bi) {
    const uint64_t rk = shfl_xor_u64(bk, kWave - 1);
    const int32_t ri = __shfl_xor(bi, kWave - 1, kWave);
    const bool r_lo = ent_less(rk, ri, ak, ai);
    uint64_t lo_k = r_lo ? rk : ak, hi_k = r_lo ? ak : rk;
    int32_t lo_i = r_lo ? ri : ai, hi_i = r_lo ? ai : ri;
    wave_merge64(lo_k, lo_i);
    wave_merge64(hi_k, hi_i);
    ak = lo_k;
    ai = lo_i;
    bk = hi_k;
    bi = hi_i;
}

// Best 256 candidates seen: chunk c (k_c / i_c) holds ranks 64 c .. 64 c + 63.
template <>
struct WaveList<256> {
    uint64_t k0, k1, k2, k3;
    int32_t i0, i1, i2, i3;
    __device__ __forceinline__ void init() {
        k0 = k1 = k2 = k3 = kKeyInvalid;
        i0 = i1 = i2 = i3 = kIdInvalid;
    }
    // (reads lane l of every chunk and selects among the values: a select among the members
    // themselves becomes a dynamically indexed stack array)
    __device__ __forceinline__ void at(int idx, uint64_t& k, int32_t& i) const {
        const int c = idx >> 6, l = idx & (kWave - 1);
        const uint64_t r0 = readlane_u64(k0, l), r1 = readlane_u64(k1, l);
        const uint64_t r2 = readlane_u64(k2, l), r3 = readlane_u64(k3, l);
        const int32_t j0 = __builtin_amdgcn_readlane(i0, l), j1 = __builtin_amdgcn_readlane(i1, l);
        const int32_t j2 = __builtin_amdgcn_readlane(i2, l), j3 = __builtin_amdgcn_readlane(i3, l);
        k = c == 0 ? r0 : c == 1 ? r1 : c == 2 ? r2 : r3;
        i = c == 0 ? j0 : c == 1 ? j1 : c == 2 ? j2 : j3;
    }
    __device__ __forceinline__ void insert(uint64_t bk, int32_t bi) {
        wave_sort64(bk, bi);
        uint64_t rk = shfl_xor_u64(bk, kWave - 1);
        int32_t ri = __shfl_xor(bi, kWave - 1, kWave);
        // Ranks 0..191 survive a 64-entry batch; ranks 192..255 become the smallest 64 of
        // (chunk 3, batch).  That chunk then bubbles down: each chunk holds entries no smaller
        // than all 64 of the chunk below it, so the largest 64 of (chunk c, carried chunk) are
        // ranks 64 c + 64 .. of the whole list.
        if (ent_less(rk, ri, k3, i3)) {
            k3 = rk;
            i3 = ri;
        }
        wave_merge64(k3, i3);
        merge_halves(k2, i2, k3, i3);
        merge_halves(k1, i1, k2, i2);
        merge_halves(k0, i0, k1, i1);
    }
};

// Chunk C (ranks 64 C .. 64 C + 63, one per lane) of a list.
template <int C, int KP>
__device__ __forceinline__ void list_chunk(const WaveList<KP>& L, uint64_t& k, int32_t& i) {
    if constexpr (C == 0) {
        k = L.k0;
        i = L.i0;
    } else if constexpr (C == 1) {
        k = L.k1;
        i = L.i1;
    } else if constexpr (C == 2) {
        k = L.k2;
        i = L.i2;
    } else {
        k = L.k3;
        i = L.i3;
    }
}

// f(std::integral_constant<int, C>) for every chunk C of a KP-entry list, in order.
template <int KP, typename F>
__device__ __forceinline__ void for_chunks(F&& f) {
    f(std::integral_constant<int, 0>{});
    if constexpr (KP >= 128) f(std::integral_constant<int, 1>{});
    if constexpr (KP == 256) {
        f(std::integral_constant<int, 2>{});
        f(std::integral_constant<int, 3>{});
    }
}

// Offers one candidate per lane; only entries that beat the current K-th entry are merged.
// Returns true (wave-uniform) when the list changed.
template <int KP>
__device__ __forceinline__ bool list_offer(WaveList<KP>& L, int K, uint64_t ck, int32_t ci) {
    uint64_t tk;
    int32_t ti;
    L.at(K - 1, tk, ti);
    const bool useful = ent_less(ck, ci, tk, ti);
    if (__ballot(useful) == 0) return false;
    L.insert(useful ? ck : kKeyInvalid, useful ? ci : kIdInvalid);
    return true;
}

// Stage Z staging area per wave: kStageCh x (kWave + 1) floats, used by refine_rows as
// kStageRows rows of kStageDims + 1 floats
constexpr int kStageCh = 32;
constexpr int kStageRows = 16, kStageDims = 128;
static_assert(kStageRows * (kStageDims + 1) <= kStageCh * (kWave + 1), "staging area");

// Canonical float64 distance of the first `nq` (1 .. 64) queued survivors (lane i <- survivor
// i), in dimension order.  Rows move in groups of 16, 128 dims (512 contiguous bytes) of each
// row at a time, every load of a group issued before the first is used, and are staged in LDS
// (row stride 129 floats: the lanes' reads of their rows fall in distinct banks).  Whole
// 512-byte runs in flight matter for a base in mapped host memory: random rows cross PCIe at
// ~51 GB/s read this way against ~40 GB/s as 128-byte pieces one 32-dim chunk at a time.
// With xb8 (the same rows as uint8, exact; D a multiple of 16, rows 16-byte aligned) the rows
// are read from it instead: 128 bytes per 128 dims, converted to float32 exactly when staged.
__device__ __forceinline__ double refine_rows(const float* __restrict__ xb,
                                              const uint8_t* __restrict__ xb8, int D,
                                              const int32_t* q_spos, int nq,
                                              float (*stage)[kWave + 1],
                                              const double* s_q64) {
    const int lane = lane_id();
    const int half = lane >> 5, kk = lane & 31;
    float* st = &stage[0][0];
    constexpr int RS = kStageDims + 1;
    const bool vec4 = (D & 3) == 0 && (reinterpret_cast<uintptr_t>(xb) & 15) == 0;
    double acc = 0.0;
    for (int g0 = 0; g0 < nq; g0 += kStageRows) {
        const int ng = min(kStageRows, nq - g0);
        const bool mine = lane >= g0 && lane < g0 + ng;
        for (int d0 = 0; d0 < D; d0 += kStageDims) {
            const int ch = min(kStageDims, D - d0);
            if (xb8) {
                // the group's rows as 16-byte pieces (16 dims each, ch / 16 per row), two per
                // lane: piece j = lane + 64 m is piece j % per of row j / per; pieces past the
                // group's rows reload its last row and are not staged
                const int per = ch >> 4;
                uint4 v8[2];
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int j = lane + kWave * m, r = j / per, p = j - r * per;
                    v8[m] = *reinterpret_cast<const uint4*>(
                        xb8 + (size_t)q_spos[g0 + min(r, ng - 1)] * D + d0 + 16 * p);
                }
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int j = lane + kWave * m, r = j / per, p = j - r * per;
                    if (r < ng) {
                        float* dst = st + r * RS + 16 * p;
                        const uint32_t w4[4] = {v8[m].x, v8[m].y, v8[m].z, v8[m].w};
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            dst[e] = (float)((w4[e >> 2] >> (8 * (e & 3))) & 0xffu);
                    }
                }
            } else if (vec4) {
                // lane (half, kk): float4 kk of rows g0 + 2 k + half; rows past the group and
                // float4s past the chunk reload the last ones (never staged)
                const int c4 = min(kk, (ch >> 2) - 1);
                float4 v[kStageRows / 2];
#pragma unroll
                for (int k = 0; k < kStageRows / 2; ++k) {
                    const int r = g0 + min(2 * k + half, ng - 1);
                    v[k] = *reinterpret_cast<const float4*>(xb + (size_t)q_spos[r] * D + d0 + 4 * c4);
                }
                if (4 * kk < ch) {
#pragma unroll
                    for (int k = 0; k < kStageRows / 2; ++k) {
                        float* dst = st + (2 * k + half) * RS + 4 * kk;
                        dst[0] = v[k].x;
                        dst[1] = v[k].y;
                        dst[2] = v[k].z;
                        dst[3] = v[k].w;
                    }
                }
            } else {
                // any D: lane (half, kk) holds dims kk, kk + 32, kk + 64, kk + 96 of its rows
                float v[kStageRows / 2][4];
#pragma unroll
                for (int k = 0; k < kStageRows / 2; ++k) {
                    const float* xr = xb + (size_t)q_spos[g0 + min(2 * k + half, ng - 1)] * D + d0;
#pragma unroll
                    for (int m = 0; m < 4; ++m) v[k][m] = xr[min(kk + 32 * m, ch - 1)];
                }
#pragma unroll
                for (int k = 0; k < kStageRows / 2; ++k)
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        if (kk + 32 * m < ch) st[(2 * k + half) * RS + kk + 32 * m] = v[k][m];
            }
            wave_sync();
            if (mine) {
                const float* sr = st + (lane - g0) * RS;
                for (int k = 0; k < ch; ++k) {
                    const double t = (double)sr[k] - s_q64[d0 + k];
                    acc = fma(t, t, acc);
                }
            }
            wave_sync();
        }
    }
    return acc;
}

}  // namespace trident
