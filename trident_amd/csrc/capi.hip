// C ABI of libtrident_hip.so (declared in include/trident_hip.h): argument validation,
// workspace carving and the launch sequence of one batched lossless IVF query.
//
// Launch sequence of trident_search (reference launch_trident_v4_search,
// src/trident_v4_kernels.cu:1172-1604):
//   prep_queries -> coarse_dist -> select_probes           (front end, :1233-1259)
//   p_init rule                                            (:1264-1276)
//   fill / count / scan / scatter pairs                    (:1279-1289)
//   pass 1: fill cand_cnt, pair_scan, merge  -> tau        (:1451-1512)
//   pass 2: fill cand_cnt, pair_scan(tau), merge -> top-K  (:1514-1575)
//   mode 0 with rerank_m > 0: merges keep the top M by acc_hat, rerank -> top-K
//                                                          (:1487-1500, :1550-1566, :1044-1170)
// Every launch goes on the caller's stream; no allocation, no host synchronisation.
// Counters are cleared with a fill kernel (no memset nodes), so the sequence can be
// captured in a graph.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/trident_hip.h"
#include "common.hpp"
#include "kernels.hpp"

using namespace trident;

// Scratch memory of trident_search_noalloc, for callers that cannot allocate: one copy of this
// array on every GPU the library runs on, held until the process ends.  Host code never uses
// the array's name as an address (on the host it is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) unsigned char scratch[TRIDENT_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once looked up

// The current device's copy of `scratch` (looked up on the first call on that device).
int scratch_of_current_device(void** ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(TRIDENT_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(TRIDENT_ERR_UNSUPPORTED, "device %d outside [0, %d)", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(TRIDENT_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return TRIDENT_OK;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(TRIDENT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return TRIDENT_OK;
}

constexpr size_t kAlign = 256;
inline size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

struct Carver {
    char* base;
    size_t off = 0;
    template <typename T>
    T* take(size_t count) {
        T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
        off = align_up(off + count * sizeof(T));
        return p;
    }
};

struct Workspace {
    double* xq64;
    double* xrot64;
    float* xrot32;
    double* qerr;
    double* cd64;
    int32_t* probe_cids;
    float* probe_dqcs;
    int32_t* counts;
    int32_t* seg_off;
    int32_t* cursor;
    int32_t* blk_tot;  // [2 * kBlock] block totals of the multi-block scans
    int32_t* pair_cids;
    int32_t* pair_qids;
    float* pair_dqcs;
    int32_t* pair_rank;              // group_pairs past the LDS histogram: arrival ranks
    uint64_t* cand_key;
    int32_t* cand_id;
    int32_t* cand_cnt;
    uint64_t* list_key;
    int32_t* list_id;
    double* tau64;
    unsigned long long* stat_slots;  // [kStatSlots, 4] telemetry partials
    int4* units;                     // [max_units] batched-route work units (both passes)
    int32_t* unit_off;               // [2 * nlist + 1]
    int32_t* unit_ctr;               // [2, 8 * kCtrStride] per-launch, per-XCD counters
    int64_t max_units;
    int2* groups;                    // [max_groups] batched-route weight groups
    int32_t* grp_off;                // [nlist + 1]
    int64_t max_groups;
    int8_t* pw;                      // [B * nprobe, 2, DP] batched-route weight planes
    PairRec* prec;                   // [B * nprobe]
    LbRec* lbr;                      // [B * nprobe]
    int2* lbk;                       // [B * nprobe] (kq, kq_pre)
    double* cbound;                  // [nlist, kCbStride]
    double* qep;                     // [B]
    uint2* ub_list;                  // [B, ub_cap] seeding bounds and rows (batched route)
    int32_t* ub_cnt;                 // [B]
    uint32_t* ub_best;               // [B]
    int32_t* seed_cnt;               // [B]
    int64_t ub_cap;
    float* qt32;                     // band front end (Dq > 128): queries, matrix-core tile layout
    uint32_t* qtb;                   // band front end (Dq <= 128): queries, bfloat16 split layout
    uint32_t* cmtb;                  // band front end (Dq <= 128): centroids, bfloat16 split layout
    float* tmin;                     // [B, ceil(nlist / 16)] tile minima (nlist >= kTileMinNlist)
    float* qn32;                     // [B] their squared norms
    float* cm32;                     // [nlist, Dq] centroid-major zero-padded centroids
    float* cmt32;                    // the centroids in the matrix-core tile layout
    float* cn32;                     // [nlist] their squared norms
    unsigned long long* cmax2;       // largest centroid squared norm (float64 bits)
    // parallel rescan of overflowed candidate lists (batched route): slots for up to ovf_max
    // queries, each with [nprobe, 128] per-probe lists
    int64_t ovf_max;
    int32_t* ovf_n;                  // [1]
    int32_t* ovf_q;                  // [ovf_max]
    int32_t* ovf_slot;               // [B]
    double* ovf_t;                   // [ovf_max]
    uint64_t* ovf_key;               // [ovf_max, nprobe, KP <= 128]
    int32_t* ovf_id;
    size_t bytes;
};

// Overflowed queries rescanned in parallel per search (the rest take the merge's serial rescan):
// 188 at B = 10,000, 18.5 MB of per-probe lists at K <= 64.  A configs[4] search whose seeding
// threshold was made loose on purpose (p_init 1) overflows fewer than that: 243 -> 17 ms per
// step against the serial rescan; larger budgets (B / 16, B / 4) changed nothing.
inline int64_t ovf_slots_of(int64_t B) { return std::min<int64_t>(B, 32 + B / 64); }

// Bytes of one batched-route weight plane: whole 64-dim steps.
inline int64_t plane_bytes(int D_pad) { return 64 * (int64_t)((D_pad + 63) / 64); }

// Candidate-list slots per query.  The batched route stores every lower-bound survivor there
// (before its exact test), so lists are at least 64 * nprobe deep (12 bytes a slot; only used
// slots are touched): a longer list makes that query's probes be rescanned (the SQ8 bounds of
// every probed row, one wave per (query, probe) for up to ovf_slots_of(B) queries, one wave per
// query past that, and the rows near the top-K refined), so the lists are sized to make that
// rare.  Past 64 neighbours in
// more than 256 dims the K-th distance sits in the bulk of the distance distribution (cfg 3,
// K = 100: ~1 % of candidates pass, ~2,300 per query with a long tail), so those lists are 8x
// deeper.  An index with a fine level keeps its base in host memory, where an overflow costs
// most, so its lists are twice as deep again.
inline int64_t cand_cap(int64_t nprobe, int64_t K, int64_t D_pad, bool fine) {
    return nprobe * std::max<int64_t>(K, 64) * (K > 64 && D_pad > 256 ? 8 : 1) * (fine ? 2 : 1);
}

Workspace carve(const TridentIndexView* ix, void* base, int64_t B, int64_t nprobe, int64_t K) {
    Carver c{static_cast<char*>(base)};
    Workspace w;
    const int64_t KP = K <= 64 ? 64 : K <= 128 ? 128 : 256;
    const int64_t cap = cand_cap(nprobe, K, ix->D_pad, ix->fine_codes && ix->fine_qp);
    w.xq64 = c.take<double>(B * ix->D);
    w.xrot64 = c.take<double>(B * ix->D_pad);
    w.xrot32 = c.take<float>(B * ix->D_pad);
    w.qerr = c.take<double>(B * ix->D_pad);
    // float64 coarse distances [B, nlist], or the band path's float32 approximations in rows of
    // band_lda(nlist) floats (never more bytes: band_lda(n) <= n + 3 floats <= 2 n for n >= 3,
    // and the rows of smaller n get the extra room here)
    w.cd64 = c.take<double>(B * std::max<int64_t>(ix->nlist, (band_lda(ix->nlist) + 1) / 2));
    w.probe_cids = c.take<int32_t>(B * nprobe);
    w.probe_dqcs = c.take<float>(B * nprobe);
    w.counts = c.take<int32_t>(2 * ((int64_t)ix->nlist + 1));
    w.seg_off = c.take<int32_t>(2 * ((int64_t)ix->nlist + 1));
    w.cursor = c.take<int32_t>(2 * ((int64_t)ix->nlist + 1));
    w.blk_tot = c.take<int32_t>(2 * kBlock);
    w.pair_cids = c.take<int32_t>(B * nprobe);
    w.pair_qids = c.take<int32_t>(B * nprobe);
    w.pair_dqcs = c.take<float>(B * nprobe);
    w.pair_rank = c.take<int32_t>(B * nprobe);
    w.cand_key = c.take<uint64_t>(B * cap);
    w.cand_id = c.take<int32_t>(B * cap);
    w.cand_cnt = c.take<int32_t>(B);
    w.list_key = c.take<uint64_t>(B * KP);
    w.list_id = c.take<int32_t>(B * KP);
    w.tau64 = c.take<double>(B);
    w.stat_slots = c.take<unsigned long long>((size_t)kStatSlots * 4);
    w.max_units = max_units_of(B * nprobe, ix->nlist);
    w.units = c.take<int4>(w.max_units);
    w.unit_off = c.take<int32_t>(2 * (int64_t)ix->nlist + 1);
    w.unit_ctr = c.take<int32_t>(2 * 8 * kCtrStride);
    w.max_groups = max_groups_of(B * nprobe, ix->nlist);
    w.groups = c.take<int2>(w.max_groups);
    w.grp_off = c.take<int32_t>((int64_t)ix->nlist + 1);
    w.pw = c.take<int8_t>(B * nprobe * 2 * plane_bytes(ix->D_pad));
    w.prec = c.take<PairRec>(B * nprobe);
    w.lbr = c.take<LbRec>(B * nprobe);
    w.lbk = c.take<int2>(B * nprobe + 32);  // + 32: the scan reads whole 32-row groups
    w.cbound = c.take<double>(kCbStride * (int64_t)ix->nlist);
    w.qep = c.take<double>(B);
    w.ub_cap = ub_cap_of(std::min<int64_t>(K, 64));
    w.ub_list = c.take<uint2>(B * w.ub_cap);
    w.ub_cnt = c.take<int32_t>(B);
    w.ub_best = c.take<uint32_t>(B);
    w.seed_cnt = c.take<int32_t>(B);
    const int64_t Dq = band_dq(ix->D);
    const int64_t Dpb = Dq <= 128 ? 32 * band_steps_bf16((int)Dq) : 0;  // bfloat16 split dims
    w.qt32 = c.take<float>(Dq > 128 ? (B + 15) / 16 * 16 * Dq : 0);
    w.qtb = c.take<uint32_t>((B + 15) / 16 * 16 * Dpb);
    w.cmtb = c.take<uint32_t>(((int64_t)ix->nlist + 15) / 16 * 16 * Dpb);
    w.tmin = c.take<float>(ix->nlist >= kTileMinNlist && Dq <= 128 ? B * (((int64_t)ix->nlist + 15) / 16) : 0);
    w.qn32 = c.take<float>(B);
    w.cm32 = c.take<float>((int64_t)ix->nlist * Dq);
    w.cmt32 = c.take<float>(((int64_t)ix->nlist + 15) / 16 * 16 * Dq);
    w.cn32 = c.take<float>(ix->nlist);
    w.cmax2 = c.take<unsigned long long>(1);
    w.ovf_max = ovf_slots_of(B);
    w.ovf_n = c.take<int32_t>(1);
    w.ovf_q = c.take<int32_t>(w.ovf_max);
    w.ovf_slot = c.take<int32_t>(B);
    w.ovf_t = c.take<double>(w.ovf_max);
    w.ovf_key = c.take<uint64_t>(w.ovf_max * nprobe * std::min<int64_t>(KP, 128));
    w.ovf_id = c.take<int32_t>(w.ovf_max * nprobe * std::min<int64_t>(KP, 128));
    w.bytes = c.off;
    return w;
}

int validate_index(const TridentIndexView* ix) {
    if (!ix) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "index view is NULL");
    if (ix->N < 0 || ix->D < 1 || ix->nlist < 1)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad index sizes N=%d D=%d nlist=%d", ix->N,
                    ix->D, ix->nlist);
    if (ix->D_pad < ix->D || ix->D_pad % 32 != 0)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "D_pad=%d must be a multiple of 32 >= D=%d",
                    ix->D_pad, ix->D);
    if (ix->seed_rows < 0)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "seed_rows=%d must be >= 0", ix->seed_rows);
    if (ix->xb_sorted_u8 && (ix->D % 16 != 0 || (reinterpret_cast<uintptr_t>(ix->xb_sorted_u8) & 15) != 0))
        return fail(TRIDENT_ERR_INVALID_ARGUMENT,
                    "xb_sorted_u8 needs D a multiple of 16 (D=%d) and a 16-byte aligned pointer", ix->D);
    if (ix->tile_size < 64 || ix->tile_size % 64 != 0)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "tile_size=%d must be a positive multiple of 64",
                    ix->tile_size);
    if (ix->num_blocks < 1 || ix->num_blocks > 64)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "num_blocks=%d outside [1, 64]", ix->num_blocks);
    if (!ix->W_combined || !ix->b_combined || !ix->cluster_vec_off || !ix->cluster_tile_off ||
        !ix->xb_sorted || !ix->tile_orig_ids)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "index view has NULL tensors");
    if (!(ix->rot_sq_min > 0.0) || !(ix->rot_sq_max >= ix->rot_sq_min))
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad rotation bounds [%g, %g]", ix->rot_sq_min,
                    ix->rot_sq_max);
    if (ix->cent_rows && (!ix->cent_tiles || !ix->cent_norms || !(ix->cent_norm_max >= 0.0) ||
                          !(ix->cent_norm_max < INFINITY)))
        return fail(TRIDENT_ERR_INVALID_ARGUMENT,
                    "cent_rows needs cent_tiles, cent_norms and a finite cent_norm_max >= 0");
    return TRIDENT_OK;
}

// The batched routes scan per-cluster counters in blocks of kBlock clusters and carry the block
// totals in one block (unit_scan_carry_kernel: 2 nlist counters, at most kBlock blocks).
constexpr int kMaxBatchedNlist = kBlock * kBlock / 2;

// The SQ8 parameters every SQ8 route reads; the reference packing (sq8_packed) only where
// `packed` (the per-pair scans, modes 0 / 1, the bound entry points).  A mode-2 index may carry
// the batched route's cells (sq8_cells) alone: choose_route then takes the batched route.
int validate_cascade_index(const TridentIndexView* ix, bool packed = true) {
    if (!ix->vmin || !ix->delta || !ix->eps_dim || !ix->blk_bounds4)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "cascade route needs the SQ8 tensors");
    if (packed && !ix->sq8_packed)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "this route reads sq8_packed, which the index view lacks");
    if (!ix->sq8_packed && !ix->sq8_cells)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "the index view holds neither sq8_packed nor sq8_cells");
    return TRIDENT_OK;
}

double rho_of(int D_pad) { return (double)(D_pad + 4) * 0x1p-24; }

ScanArgs make_scan_args(const TridentIndexView* ix, const Workspace& w, int K, int64_t cap,
                        int use_l1, unsigned long long* stats) {
    ScanArgs a{};
    a.sq8 = ix->sq8_packed;
    a.tile_oids = ix->tile_orig_ids;
    a.tile_rmm = ix->tile_r_minmax;
    a.tile_off = ix->cluster_tile_off;
    a.vec_off = ix->cluster_vec_off;
    a.xb = ix->xb_sorted;
    a.vmin = ix->vmin;
    a.delta = ix->delta;
    a.eps = ix->eps_dim;
    a.blk = ix->blk_bounds4;
    a.D = ix->D;
    a.D_pad = ix->D_pad;
    a.T = ix->tile_size;
    a.nb = ix->num_blocks;
    a.per_cluster = ix->per_cluster_sq8;
    a.use_l1 = use_l1;
    a.xq64 = w.xq64;
    a.xrot64 = w.xrot64;
    a.qerr = w.qerr;
    a.cand_key = w.cand_key;
    a.cand_id = w.cand_id;
    a.cand_cnt = w.cand_cnt;
    a.cap = (int)cap;
    a.K = K;
    a.stats = stats;
    const double rho = rho_of(ix->D_pad);
    a.lb_scale = ix->rot_sq_max * (1.0 + rho) * (1.0 + 1e-12);
    a.ub_scale = (1.0 + rho) * (1.0 + 1e-12) / ix->rot_sq_min;
    return a;
}

template <int KP, int KIND>
int launch_scan(const ScanArgs& a, hipStream_t st) {
    if (a.M <= 0) return TRIDENT_OK;
    const size_t dyn = scan_dyn_lds_bytes(a.D, a.D_pad);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)pair_scan_kernel<KP, KIND>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e != hipSuccess)
            return fail(TRIDENT_ERR_HIP, "hipFuncSetAttribute(pair_scan): %s", hipGetErrorString(e));
        attr_set = true;
    }
    const unsigned nx = (unsigned)((a.M + 7) / 8);
    pair_scan_kernel<KP, KIND><<<dim3(nx * 8), dim3(kBlock), dyn, st>>>(a);
    return check_launch("pair_scan_kernel");
}

template <int KO>
int launch_rerank(const RerankArgs& r, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)rerank_kernel<KO>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        if (e != hipSuccess)
            return fail(TRIDENT_ERR_HIP, "hipFuncSetAttribute(rerank): %s", hipGetErrorString(e));
        attr_set = true;
    }
    rerank_kernel<KO><<<(unsigned)r.B, kBlock, (size_t)r.D * sizeof(double), st>>>(r);
    return check_launch("rerank_kernel");
}

// Mode 0 reranks the top M = min(max(rerank_m, K), 200) entries by acc_hat (reference
// :1439-1444, :1071-1073); its merged lists hold max(K, M) entries, every other mode's K.
inline int64_t rerank_len(int mode, int64_t K, int64_t rerank_m) {
    return mode == TRIDENT_MODE_SQ8_RERANK && rerank_m > 0
               ? std::min<int64_t>(std::max<int64_t>(rerank_m, K), 200) : 0;
}
inline int64_t merged_list_len(int mode, int64_t K, int64_t rerank_m) {
    return std::max<int64_t>(K, rerank_len(mode, K, rerank_m));
}

inline int list_kp(int64_t k) { return k <= 64 ? 64 : k <= 128 ? 128 : 256; }

// One per-pair pass with a.K entries per pair (a.K <= 128, or <= 256 for kScanHat).
int dispatch_scan(const ScanArgs& a, int kind, hipStream_t st) {
    const int kp = list_kp(a.K);
    switch (kind) {
        case kScanCascade:
            return kp == 64 ? launch_scan<64, kScanCascade>(a, st) : launch_scan<128, kScanCascade>(a, st);
        case kScanCascadeUb:
            return kp == 64 ? launch_scan<64, kScanCascadeUb>(a, st)
                            : launch_scan<128, kScanCascadeUb>(a, st);
        case kScanExact:
            return kp == 64 ? launch_scan<64, kScanExact>(a, st) : launch_scan<128, kScanExact>(a, st);
        case kScanTribase:
            return kp == 64 ? launch_scan<64, kScanTribase>(a, st) : launch_scan<128, kScanTribase>(a, st);
        case kScanHat:
            return kp == 64    ? launch_scan<64, kScanHat>(a, st)
                   : kp == 128 ? launch_scan<128, kScanHat>(a, st)
                               : launch_scan<256, kScanHat>(a, st);
        default:
            return fail(TRIDENT_ERR_UNSUPPORTED, "scan kind %d", kind);
    }
}

// Route of a mode-2 search.  The batched route needs the per-vector scalars, K <= 128 (a
// seeding unit lists at most 64 bounds per query; the threshold is the K-th over all of a
// query's units and the merge keeps 128), D_pad <= 1024 (query weights
// held in registers: 8 VGPRs per 64 dims) and N < 2^27 (a queued survivor packs its index within the cluster
// into 28 bits); AUTO takes it when clusters are shared by >= 8 queries on average, where
// the contraction is dense enough for the matrix cores.
int choose_route(const TridentIndexView* ix, const TridentSearchParams* sp, int B, int K,
                 int nprobe, int* route) {
    const bool ok = ix->vec_Ar && ix->sq8_cells && ix->orig_ids_sorted && K <= 128 &&
                    ix->D_pad <= 1024 && ix->nlist <= kMaxBatchedNlist &&
                    ix->N < (1 << 27) &&
                    max_units_of((int64_t)B * nprobe, ix->nlist) < 0x7fffffff;
    // an index without the reference packing (sq8_packed) has only the batched route
    const bool pair_ok = ix->sq8_packed != nullptr;
    switch (sp->route) {
        case TRIDENT_ROUTE_PAIR:
            if (!pair_ok)
                return fail(TRIDENT_ERR_UNSUPPORTED,
                            "the per-pair route reads sq8_packed, which the index view lacks");
            *route = TRIDENT_ROUTE_PAIR;
            return TRIDENT_OK;
        case TRIDENT_ROUTE_BATCHED:
            if (!ok)
                return fail(TRIDENT_ERR_UNSUPPORTED,
                            "batched route needs vec_Ar, sq8_cells, K <= 128, D_pad <= 1024, "
                            "nlist <= %d and N < 2^27 (K=%d, D_pad=%d, nlist=%d, N=%d)",
                            kMaxBatchedNlist, K, ix->D_pad, ix->nlist, ix->N);
            *route = TRIDENT_ROUTE_BATCHED;
            return TRIDENT_OK;
        case TRIDENT_ROUTE_AUTO:
            if (!pair_ok && !ok)
                return fail(TRIDENT_ERR_UNSUPPORTED,
                            "the index view lacks sq8_packed (per-pair route) and this search "
                            "cannot take the batched route (K=%d, D_pad=%d, N=%d)",
                            K, ix->D_pad, ix->N);
            *route = (ok && (!pair_ok || (double)B * nprobe >= 8.0 * ix->nlist))
                         ? TRIDENT_ROUTE_BATCHED
                         : TRIDENT_ROUTE_PAIR;
            return TRIDENT_OK;
        default:
            return fail(TRIDENT_ERR_INVALID_ARGUMENT, "route=%d outside {0,1,2}", sp->route);
    }
}

// Slices of each seeding cluster the seeding pass (and mode 10's warm-up) scans: the first one
// while K <= 64 and rows are cheap to refine (base in HBM, or a fine level in front of a host
// base), else the first two.  A seeding threshold from fewer rows is looser: with K <= 50 and
// such a base one slice is faster (configs[4] 7.25 -> 7.17 ms, configs[3] K = 10 1.66 -> 1.57
// ms), but at K = 100 (configs[2] 5.5 -> 7.5 ms, configs[3] 3.0 ms -> overflowed candidate
// lists) and for a host base without a fine level (every extra survivor crosses PCIe) it is not.
inline int seed_slice_count(int K, bool xb_host, bool fine) {
    return K <= 64 && (!xb_host || fine) ? 1 : 2;
}

// Mode 10: the matrix-core cluster-major scan (cm_scan_kernel, cm_scan_wide_kernel past 256
// dims) or the per-pair float64 scan.  Both read every probed row from the base; the matrix-core
// route reads a row once per unit (up to 64 queries of its cluster) instead of once per (query,
// probe) pair.  It needs D_pad <= 1024 (the refine's query row in LDS) and K <= 128 (the
// merge's lists).  AUTO takes it when clusters are shared by at least 4 queries on average
// (16-row tiles with fewer rows leave most of each matrix instruction idle), and always for a
// base in mapped host memory (every row read crosses PCIe, and this route reads fewer).
int choose_cm_route(const TridentIndexView* ix, const TridentSearchParams* sp, int B, int K,
                    int nprobe, bool xb_host, bool* cm) {
    const bool ok = ix->orig_ids_sorted && K <= 128 && ix->D_pad <= 1024 &&
                    ix->nlist <= kMaxBatchedNlist && ix->N < (1 << 27) &&
                    max_units_of((int64_t)B * nprobe, ix->nlist) < 0x7fffffff;
    switch (sp->route) {
        case TRIDENT_ROUTE_PAIR:
            *cm = false;
            return TRIDENT_OK;
        case TRIDENT_ROUTE_BATCHED:
            if (!ok)
                return fail(TRIDENT_ERR_UNSUPPORTED,
                            "mode 10 batched route needs orig_ids_sorted, K <= 128, D_pad <= "
                            "1024, nlist <= %d and N < 2^27 (K=%d, D_pad=%d, nlist=%d, N=%d)",
                            kMaxBatchedNlist, K, ix->D_pad, ix->nlist, ix->N);
            *cm = true;
            return TRIDENT_OK;
        case TRIDENT_ROUTE_AUTO:
            *cm = ok && (xb_host || (double)B * nprobe >= 4.0 * ix->nlist);
            return TRIDENT_OK;
        default:
            return fail(TRIDENT_ERR_INVALID_ARGUMENT, "route=%d outside {0,1,2}", sp->route);
    }
}

template <int D4>
const void* cm_kernel_ptr() {
    return reinterpret_cast<const void*>(&cm_scan_kernel<D4>);
}

// Resident grid of cm_scan_kernel<D4> (CUs x occupancy), cached per device and variant.
template <int D4>
unsigned cm_grid() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int cu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cu < 1)
            cu = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, cm_kernel_ptr<D4>(), kBlock, 0) !=
                hipSuccess ||
            per_cu < 1)
            per_cu = 2;
        cached[dev] = std::max(8, cu * per_cu);
    }
    return (unsigned)cached[dev];
}

// Resident grid of cm_scan_wide_kernel, cached per device.
unsigned cm_wide_grid() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int cu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cu < 1)
            cu = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void*>(&cm_scan_wide_kernel), kBlock, 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 2;
        cached[dev] = std::max(8, cu * per_cu);
    }
    return (unsigned)cached[dev];
}

template <int D4 = 8>
int launch_cm(const BatchArgs& b, hipStream_t st) {
    if constexpr (D4 > 64) {
        if (b.D_pad > 1024)
            return fail(TRIDENT_ERR_UNSUPPORTED, "mode 10 batched route needs D_pad <= 1024");
        cm_scan_wide_kernel<<<cm_wide_grid(), kBlock, 0, st>>>(b);
        return check_launch("cm_scan_wide_kernel");
    } else {
        if (b.D_pad != 4 * D4) return launch_cm<D4 + 8>(b, st);
        cm_scan_kernel<D4><<<cm_grid<D4>(), kBlock, 0, st>>>(b);
        return check_launch("cm_scan_kernel");
    }
}

// Seeding pass: ub_scan_kernel<KS, M> (M = per-lane list length, 4 when K <= 16);
// lower-bound pass: lb_scan_kernel<KS> (D_pad <= 256) or lb_scan_wide_kernel<KS>.
template <bool UB, int KS, int M>
const void* batch_kernel_ptr() {
    if constexpr (UB) return reinterpret_cast<const void*>(&ub_scan_kernel<KS, M>);
    else if constexpr (KS <= 4) return reinterpret_cast<const void*>(&lb_scan_kernel<KS>);
    else return reinterpret_cast<const void*>(&lb_scan_wide_kernel<KS>);
}

// Queries per lower-bound unit: 128 on the narrow layout (four waves of 32), 64 on the wide
// layout (four waves of 16).
inline int lb_unit_q(int D_pad) { return D_pad <= 256 ? kUnitQ : kUnitQWide; }

// Persistent grid of a batched-scan variant: as many workgroups as are resident at once (CUs x
// the occupancy its registers and LDS allow), rounded to a multiple of 8 so every XCD gets the
// same number; cached per device and variant.
template <bool UB, int KS, int M>
unsigned persistent_grid() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int cu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cu < 1)
            cu = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, batch_kernel_ptr<UB, KS, M>(),
                                                         kBlock, 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 2;
        cached[dev] = std::max(8, ((cu * per_cu + 7) / 8) * 8);
    }
    return (unsigned)cached[dev];
}

template <bool UB, int KS>
int launch_batch_ks(const BatchArgs& b, hipStream_t st) {
    if constexpr (UB) {
        if (b.K <= 16)
            ub_scan_kernel<KS, 4><<<persistent_grid<true, KS, 4>(), kBlock, 0, st>>>(b);
        else
            ub_scan_kernel<KS, 16><<<persistent_grid<true, KS, 16>(), kBlock, 0, st>>>(b);
        return check_launch("ub_scan_kernel");
    } else if constexpr (KS <= 4) {
        lb_scan_kernel<KS><<<persistent_grid<false, KS, 0>(), kBlock, 0, st>>>(b);
        return check_launch("lb_scan_kernel");
    } else {
        lb_scan_wide_kernel<KS><<<persistent_grid<false, KS, 0>(), kBlock, 0, st>>>(b);
        return check_launch("lb_scan_wide_kernel");
    }
}

// Calls f(std::integral_constant<int, KS>) for the 64-dim step count KS in [1, 16] (D_pad up
// to 1024); false for any other count.
template <int KS = 1, class F>
bool with_ks(int ks, F&& f) {
    if constexpr (KS > 16) {
        return false;
    } else {
        if (ks == KS) {
            f(std::integral_constant<int, KS>{});
            return true;
        }
        return with_ks<KS + 1>(ks, f);
    }
}

int launch_pair_prep(const BatchArgs& b, hipStream_t st) {
    if (b.M <= 0) return TRIDENT_OK;
    static_assert(kGroupQ * 2 == kWave, "one weight group per wave, 2 lanes a pair");
    // one group per wave; waves past the group count return
    const unsigned grid = (unsigned)((b.max_groups + kWavesPerBlock - 1) / kWavesPerBlock);
    const bool ok = with_ks(b.DP / 64, [&](auto ks_c) {
        pair_prep_kernel<decltype(ks_c)::value><<<grid, kBlock, 0, st>>>(b);
    });
    if (!ok) return fail(TRIDENT_ERR_UNSUPPORTED, "batched route needs D_pad <= 1024");
    return check_launch("pair_prep_kernel");
}

template <bool UB>
int launch_batch(const BatchArgs& b, hipStream_t st) {
    int rc = TRIDENT_OK;
    const bool ok = with_ks((b.D_pad + 63) / 64, [&](auto ks_c) {
        rc = launch_batch_ks<UB, decltype(ks_c)::value>(b, st);
    });
    return ok ? rc : fail(TRIDENT_ERR_UNSUPPORTED, "batched route needs D_pad <= 1024");
}

int launch_merge(const MergeArgs& m, int KP, hipStream_t st) {
    const unsigned grid = (unsigned)((m.B + kWavesPerBlock - 1) / kWavesPerBlock);
    // the bounded rescan stages 3 D_pad floats per wave (<= 48 KiB at D_pad 1024)
    const size_t dyn = m.ovf_bounds ? (size_t)kWavesPerBlock * 3 * m.D_pad * sizeof(float) : 0;
    if (KP == 64)
        merge_kernel<64><<<grid, kBlock, dyn, st>>>(m);
    else if (KP == 128)
        merge_kernel<128><<<grid, kBlock, dyn, st>>>(m);
    else
        merge_kernel<256><<<grid, kBlock, dyn, st>>>(m);
    return check_launch("merge_kernel");
}

int fill(int32_t* p, int32_t v, int64_t n, hipStream_t st) {
    if (n <= 0) return TRIDENT_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    fill_i32_kernel<<<(unsigned)blocks, 256, 0, st>>>(p, v, n);
    return check_launch("fill_i32_kernel");
}

// Writes the probes to w.probe_cids / w.probe_dqcs (row stride nprobe) and, when non-null,
// mirrors them into the caller's probe_cids / probe_dqcs (row stride ld).
int run_front_end(const TridentIndexView* ix, const float* xq, int B, int nprobe, bool rotate,
                  const Workspace& w, int32_t* probe_cids, float* probe_dqcs, int ld,
                  hipStream_t st) {
    const int ldw = ix->nlist + ix->D_pad;
    const int cols = std::max(ix->D, rotate ? ix->D_pad : 0);
    prep_queries_kernel<<<dim3((cols + 127) / 128, (B + 4 * kPrepQB - 1) / (4 * kPrepQB)),
                          dim3(64, 4), 0, st>>>(
        xq, B, ix->D, ix->D_pad, ix->W_combined, ldw, ix->nlist, ix->b_combined, w.xq64,
        w.xrot64, w.xrot32, w.qerr, rotate ? 1 : 0);
    int rc = check_launch("prep_queries_kernel");
    if (rc) return rc;
    if (nprobe <= 128) {  // band front end
        const int Dq = band_dq(ix->D);
        const float *cm = ix->cent_rows, *cmt = ix->cent_tiles, *cn = ix->cent_norms;
        const unsigned long long* cmax_dev = nullptr;
        if (!cm) {  // derive the centroid layouts into the workspace
            fill_u64_kernel<<<1, 64, 0, st>>>(w.cmax2, 0ull, 1);
            if ((rc = check_launch("fill_u64_kernel"))) return rc;
            pad_centroids_kernel<<<(unsigned)((ix->nlist + 63) / 64), 256, 0, st>>>(
                ix->W_combined, ldw, ix->nlist, ix->D, Dq, w.cm32, w.cmt32, w.cn32, w.cmax2);
            if ((rc = check_launch("pad_centroids_kernel"))) return rc;
            cm = w.cm32;
            cmt = w.cmt32;
            cn = w.cn32;
            cmax_dev = w.cmax2;
        }
        const bool split = Dq <= 128;  // bfloat16 split operands, else float32
        const int NS = split ? band_steps_bf16(Dq) : 0;
        pad_queries_kernel<<<(unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock), kBlock, 0,
                             st>>>(xq, B, ix->D, Dq, split ? nullptr : w.qt32, w.qn32, NS,
                                   split ? reinterpret_cast<uint16_t*>(w.qtb) : nullptr);
        if ((rc = check_launch("pad_queries_kernel"))) return rc;
        float* a32 = reinterpret_cast<float*>(w.cd64);  // [B, nlist] approximations
        // the streaming selector's tile minima (bfloat16 pass, from kTileMinNlist centroids)
        float* tmin = ix->nlist >= kTileMinNlist && split ? w.tmin : nullptr;
        if (split) {
            const int64_t npair = ((int64_t)ix->nlist + 15) / 16 * 16 * 16 * NS;
            centroid_bf16_kernel<<<(unsigned)std::min<int64_t>((npair + 255) / 256, 4096), 256, 0,
                                   st>>>(cm, ix->nlist, Dq, NS, w.cmtb);
            if ((rc = check_launch("centroid_bf16_kernel"))) return rc;
            const int64_t nst = ((ix->nlist + 15) / 16 + kStageTiles - 1) / kStageTiles;
            const int64_t spx = (nst + 7) / 8, nqb = (B + 63) / 64;
            const int64_t want = std::min<int64_t>(spx, std::max<int64_t>(1, kStreamBlocks / (8 * nqb)));
            const int64_t run_stages = (spx + want - 1) / want, nrun = (spx + run_stages - 1) / run_stages;
            const dim3 sgrid((unsigned)(8 * nqb * nrun));
            switch (NS) {
#define TRIDENT_GEMM_CASE(NSV)                                                                  \
    case NSV:                                                                                   \
        coarse_gemm_bf16_kernel<NSV><<<sgrid, kBlock, 0, st>>>(w.qtb, w.qn32, B, w.cmtb, cn,       \
                                                               ix->nlist, (int)run_stages, a32, tmin); \
        break;
                TRIDENT_GEMM_CASE(1) TRIDENT_GEMM_CASE(2) TRIDENT_GEMM_CASE(3) TRIDENT_GEMM_CASE(4)
#undef TRIDENT_GEMM_CASE
                default:
                    return fail(TRIDENT_ERR_INVALID_ARGUMENT, "coarse GEMM: Dq=%d", (int)Dq);
            }
            if ((rc = check_launch("coarse_gemm_bf16_kernel"))) return rc;
        } else {
            const int64_t ncg = (ix->nlist + 16 * kGemmTiles - 1) / (16 * kGemmTiles);
            coarse_gemm_kernel<<<(unsigned)(8 * ((B + 63) / 64) * ((ncg + 7) / 8)), kBlock, 0, st>>>(
                w.qt32, w.qn32, B, cmt, cn, ix->nlist, Dq, a32);
            if ((rc = check_launch("coarse_gemm_kernel"))) return rc;
        }
        const double kappa = split ? band_kappa_bf16(Dq) : band_kappa_f32(Dq);
        const double kabs = split ? band_kabs_bf16(Dq) : 0.0;
        const unsigned grid = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
        const int V = ix->nlist <= 1024 ? 16 : ix->nlist <= kBandMaxNlist ? 32 : 0;
#define TRIDENT_BAND_LAUNCH(KPV, VV, SS)                                                         \
    select_band_kernel<KPV, VV, SS><<<grid, kBlock, 0, st>>>(                                   \
        a32, w.xq64, cm, cmax_dev, ix->cent_norm_max, B, ix->nlist, ix->D, Dq, kappa, kabs,     \
        SS ? tmin : nullptr, split ? band_lda(ix->nlist) : ix->nlist, nprobe,                    \
        w.probe_cids,                                                                           \
        w.probe_dqcs, nprobe, probe_cids, probe_dqcs, ld)
        if (nprobe <= 64) {
            if (V == 16) TRIDENT_BAND_LAUNCH(64, 16, false);
            else if (V == 32) TRIDENT_BAND_LAUNCH(64, 32, false);
            else TRIDENT_BAND_LAUNCH(64, 8, true);
        } else {
            if (V == 16) TRIDENT_BAND_LAUNCH(128, 16, false);
            else if (V == 32) TRIDENT_BAND_LAUNCH(128, 32, false);
            else TRIDENT_BAND_LAUNCH(128, 8, true);
        }
#undef TRIDENT_BAND_LAUNCH
        return check_launch("select_band_kernel");
    }
    constexpr int qpb = kCoarseQW * kWavesPerBlock;
    coarse_dist_kernel<<<dim3((ix->nlist + 64 * kCoarseNC - 1) / (64 * kCoarseNC),
                                 (B + qpb - 1) / qpb),
                            kBlock, 0, st>>>(
        w.xq64, B, ix->D, ix->W_combined, ldw, ix->nlist, w.cd64);
    if ((rc = check_launch("coarse_dist_kernel"))) return rc;
    if (nprobe <= 128) {  // one wave per query, register list
        const unsigned grid = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
        if (nprobe <= 64)
            select_probes_wave_kernel<64><<<grid, kBlock, 0, st>>>(
                w.cd64, B, ix->nlist, nprobe, w.probe_cids, w.probe_dqcs, nprobe, probe_cids,
                probe_dqcs, ld);
        else
            select_probes_wave_kernel<128><<<grid, kBlock, 0, st>>>(
                w.cd64, B, ix->nlist, nprobe, w.probe_cids, w.probe_dqcs, nprobe, probe_cids,
                probe_dqcs, ld);
        return check_launch("select_probes_wave_kernel");
    }
    // nprobe > 128: the radix selector keeps a query's nlist float64 keys in LDS
    if ((int64_t)ix->nlist * 8 > 150 * 1024)
        return fail(TRIDENT_ERR_UNSUPPORTED,
                    "nprobe=%d > 128 needs nlist <= 19200 (the LDS probe selector); nlist=%d",
                    nprobe, ix->nlist);
    const size_t dyn = (size_t)ix->nlist * sizeof(uint64_t);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)select_probes_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        if (e != hipSuccess)
            return fail(TRIDENT_ERR_HIP, "hipFuncSetAttribute(select): %s", hipGetErrorString(e));
        attr_set = true;
    }
    select_probes_kernel<<<B, kBlock, dyn, st>>>(w.cd64, ix->nlist, nprobe, w.probe_cids,
                                                 w.probe_dqcs, nprobe, probe_cids, probe_dqcs,
                                                 ld);
    return check_launch("select_probes_kernel");
}

// Pair counting and scattering: LDS-aggregated per chunk while the 2 (nlist + 1) counters fit
// 64 KiB of LDS, one global atomic per pair otherwise.
int launch_count_pairs(const int32_t* probe_cids, int ld, int B, int nprobe, int p_init,
                       int nlist, int32_t* counts, hipStream_t st) {
    const int64_t total = (int64_t)B * nprobe;
    if (group_lds_bytes(nlist) <= 64 * 1024) {
        const unsigned blocks = (unsigned)((total + kGroupChunk - 1) / kGroupChunk);
        count_pairs_lds_kernel<<<blocks, kBlock, group_lds_bytes(nlist), st>>>(
            probe_cids, ld, B, nprobe, p_init, nlist, counts);
        return check_launch("count_pairs_lds_kernel");
    }
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    count_pairs_kernel<<<blocks, 256, 0, st>>>(probe_cids, ld, B, nprobe, p_init, nlist, counts);
    return check_launch("count_pairs_kernel");
}

int launch_scatter_pairs(const int32_t* probe_cids, const float* probe_dqcs, int ld, int B,
                         int nprobe, int p_init, int nlist, int32_t* cursor, int32_t* p1c,
                         int32_t* p1q, float* p1d, int32_t* p2c, int32_t* p2q, float* p2d,
                         hipStream_t st) {
    const int64_t total = (int64_t)B * nprobe;
    if (group_lds_bytes(nlist) <= 64 * 1024) {
        const unsigned blocks = (unsigned)((total + kGroupChunk - 1) / kGroupChunk);
        scatter_pairs_lds_kernel<<<blocks, kBlock, group_lds_bytes(nlist), st>>>(
            probe_cids, probe_dqcs, ld, B, nprobe, p_init, nlist, cursor, p1c, p1q, p1d, p2c, p2q,
            p2d);
        return check_launch("scatter_pairs_lds_kernel");
    }
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    scatter_pairs_kernel<<<blocks, 256, 0, st>>>(probe_cids, probe_dqcs, ld, B, nprobe, p_init,
                                                 nlist, cursor, p1c, p1q, p1d, p2c, p2q, p2d);
    return check_launch("scatter_pairs_kernel");
}

// joint = false: each pass's pairs grouped by cluster in its own array (p1*, p2*), seg_off =
// [2, nlist + 1] per-pass segment offsets (the per-pair route).  With a rank buffer (B * nprobe)
// and counters past the LDS histogram, the count keeps each pair's rank in its bin and the
// scatter needs no atomics.  joint = true: one cluster-major
// array (p1* and p2* the same array), each cluster's pass-1 pairs before its pass-2 pairs,
// seg_off rows = cluster starts and pass-2 starts (the batched route).
int group_pairs(const int32_t* probe_cids, const float* probe_dqcs, int ld, int B, int nprobe,
                int p_init, int nlist, int32_t* counts, int32_t* seg_off, int32_t* cursor,
                int32_t* p1c, int32_t* p1q, float* p1d, int32_t* p2c, int32_t* p2q, float* p2d,
                bool joint, int32_t* blk_tot, int32_t* rank, hipStream_t st) {
    int rc = fill(counts, 0, 2 * ((int64_t)nlist + 1), st);
    if (rc) return rc;
    const bool ranked = rank && group_lds_bytes(nlist) > 64 * 1024;
    const int64_t total = (int64_t)B * nprobe;
    const unsigned gblocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    if (ranked) {
        count_pairs_rank_kernel<<<gblocks, 256, 0, st>>>(probe_cids, ld, B, nprobe, p_init, nlist,
                                                         counts, rank);
        if ((rc = check_launch("count_pairs_rank_kernel"))) return rc;
    } else if ((rc = launch_count_pairs(probe_cids, ld, B, nprobe, p_init, nlist, counts, st))) {
        return rc;
    }
    if (joint) {
        // nlist <= kMaxBatchedNlist (choose_route), so the block totals fit one block's scan
        const int nblk = (nlist + kBlock - 1) / kBlock;
        scan_pairs_joint_local_kernel<<<nblk, kBlock, 0, st>>>(counts, nlist, seg_off, blk_tot);
        if ((rc = check_launch("scan_pairs_joint_local_kernel"))) return rc;
        scan_pairs_joint_carry_kernel<<<nblk, kBlock, 0, st>>>(counts, nlist, blk_tot, nblk,
                                                               seg_off, cursor);
        if ((rc = check_launch("scan_pairs_joint_carry_kernel"))) return rc;
    } else {
        scan_pairs_kernel<<<2, kBlock, 0, st>>>(counts, nlist, seg_off, cursor);
        if ((rc = check_launch("scan_pairs_kernel"))) return rc;
    }
    if (ranked) {
        scatter_pairs_rank_kernel<<<gblocks, 256, 0, st>>>(probe_cids, probe_dqcs, ld, B, nprobe,
                                                           p_init, nlist, seg_off, rank, p1c, p1q,
                                                           p1d, p2c, p2q, p2d);
        return check_launch("scatter_pairs_rank_kernel");
    }
    return launch_scatter_pairs(probe_cids, probe_dqcs, ld, B, nprobe, p_init, nlist, cursor, p1c,
                                p1q, p1d, p2c, p2q, p2d, st);
}

}  // namespace

extern "C" {

int trident_abi_version(void) { return TRIDENT_ABI_VERSION; }

const char* trident_last_error(void) { return g_last_error.c_str(); }

int32_t trident_p_init_rule(int32_t mode, int32_t B, int32_t K, int32_t nprobe,
                            int32_t rerank_m) {
    if (mode == TRIDENT_MODE_SQ8_RERANK) {
        if (nprobe <= 1 || (B == 1 && rerank_m == 0)) return 0;
        if ((rerank_m > 20 || K > 10) && nprobe >= 4) return 2;
        return 1;
    }
    if (mode != TRIDENT_MODE_CASCADE && mode != TRIDENT_MODE_SQ8 && mode != TRIDENT_MODE_TRIBASE)
        return 0;
    if (nprobe <= 1) return 0;
    if (B == 1 && K <= 10) return 1;
    if (nprobe <= 16) return 2;
    return 3;
}

int32_t trident_route_for(const TridentIndexView* ix, int32_t B, int32_t K, int32_t nprobe,
                          int32_t requested_route) {
    if (!ix) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "index view is NULL");
    TridentSearchParams sp{};
    sp.route = requested_route;
    int route = TRIDENT_ROUTE_PAIR;
    const int rc = choose_route(ix, &sp, B, K, nprobe, &route);
    return rc ? -rc : route;
}

int32_t trident_route_for_mode(const TridentIndexView* ix, int32_t mode, int32_t B, int32_t K,
                               int32_t nprobe, int32_t requested_route) {
    if (!ix) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "index view is NULL");
    if (mode == TRIDENT_MODE_CASCADE) return trident_route_for(ix, B, K, nprobe, requested_route);
    if (mode != TRIDENT_MODE_CM_EXACT) return TRIDENT_ROUTE_PAIR;
    TridentSearchParams sp{};
    sp.route = requested_route;
    bool xb_host = false;
    {
        hipPointerAttribute_t pa;
        xb_host = hipPointerGetAttributes(&pa, ix->xb_sorted) == hipSuccess &&
                  pa.type == hipMemoryTypeHost;
        (void)hipGetLastError();
    }
    bool cm = false;
    const int rc = choose_cm_route(ix, &sp, B, K, nprobe, xb_host, &cm);
    return rc ? -rc : (cm ? TRIDENT_ROUTE_BATCHED : TRIDENT_ROUTE_PAIR);
}

size_t trident_workspace_bytes(const TridentIndexView* ix, int32_t max_B, int32_t max_nprobe,
                               int32_t max_K) {
    if (!ix || max_B < 0 || max_nprobe < 1 || max_K < 1) return 0;
    return carve(ix, nullptr, max_B, max_nprobe, max_K).bytes;
}

int trident_coarse_probe(const TridentIndexView* ix, const float* xq, int32_t B, int32_t nprobe,
                         void* workspace, size_t workspace_bytes, int32_t* probe_cids,
                         float* probe_dqcs, int32_t probe_ld, void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if (B < 0 || nprobe < 1 || nprobe > ix->nlist || nprobe > 512 || probe_ld < nprobe ||
        !probe_cids || (B > 0 && !xq))
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad probe arguments B=%d nprobe=%d ld=%d", B,
                    nprobe, probe_ld);
    if (B == 0) return TRIDENT_OK;
    Workspace w = carve(ix, workspace, B, nprobe, 1);
    if (!workspace || workspace_bytes < w.bytes)
        return fail(TRIDENT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu < %zu bytes", workspace_bytes,
                    w.bytes);
    return run_front_end(ix, xq, B, nprobe, false, w, probe_cids, probe_dqcs, probe_ld,
                         static_cast<hipStream_t>(stream));
}

int trident_group_pairs(const int32_t* probe_cids, int32_t probe_ld, int32_t B, int32_t nprobe,
                        int32_t p_init, int32_t nlist, int32_t* p1_cids, int32_t* p1_qids,
                        int32_t* p2_cids, int32_t* p2_qids, int32_t* seg_off,
                        int32_t* counts_ws, void* stream) {
    if (B < 0 || nprobe < 1 || p_init < 0 || p_init > nprobe || nlist < 1 || probe_ld < nprobe ||
        !seg_off || !counts_ws || (int64_t)B * nprobe > 0x7fffffff)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad group_pairs arguments");
    if (B == 0) return TRIDENT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // cursor reuses counts_ws after the scan has consumed the counts.
    int rc = fill(counts_ws, 0, 2 * ((int64_t)nlist + 1), st);
    if (rc) return rc;
    if ((rc = launch_count_pairs(probe_cids, probe_ld, B, nprobe, p_init, nlist, counts_ws, st)))
        return rc;
    scan_pairs_kernel<<<2, kBlock, 0, st>>>(counts_ws, nlist, seg_off, seg_off);
    if ((rc = check_launch("scan_pairs_kernel"))) return rc;
    // seg_off now doubles as the cursor; restore it from the counts afterwards.
    if ((rc = launch_scatter_pairs(probe_cids, nullptr, probe_ld, B, nprobe, p_init, nlist, seg_off,
                                   p1_cids, p1_qids, nullptr, p2_cids, p2_qids, nullptr, st)))
        return rc;
    scan_pairs_kernel<<<2, kBlock, 0, st>>>(counts_ws, nlist, seg_off, seg_off);
    return check_launch("scan_pairs_kernel");
}

int trident_search(const TridentIndexView* ix, const TridentSearchParams* sp, const float* xq,
                   void* workspace, size_t workspace_bytes, const TridentSearchOutputs* out,
                   void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if (!sp || !out) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "params/outputs are NULL");
    const int mode = sp->mode, B = sp->B, K = sp->K, nprobe = sp->nprobe;
    if (mode != TRIDENT_MODE_CASCADE && mode != TRIDENT_MODE_CM_EXACT &&
        mode != TRIDENT_MODE_TRIBASE && mode != TRIDENT_MODE_SQ8 && mode != TRIDENT_MODE_SQ8_RERANK)
        return fail(TRIDENT_ERR_UNSUPPORTED,
                    "mode %d is not supported (0 = SQ8 + rerank, 1 = SQ8, 2 = cascade, 10 = "
                    "cluster-major exact, 11 = Tribase)", mode);
    if (sp->rerank_m < 0) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "rerank_m=%d", sp->rerank_m);
    if (B < 0) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "B=%d", B);
    if (K < 1 || K > 128) return fail(TRIDENT_ERR_UNSUPPORTED, "K=%d outside [1, 128]", K);
    if (nprobe < 1 || nprobe > ix->nlist || nprobe > 512)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "nprobe=%d outside [1, min(nlist=%d, 512)]",
                    nprobe, ix->nlist);
    if ((int64_t)B * nprobe > 0x7fffffff)
        return fail(TRIDENT_ERR_UNSUPPORTED, "B * nprobe = %lld exceeds 2^31 - 1",
                    (long long)B * nprobe);
    if (sp->ub_seed < 0 || sp->ub_seed > 2)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "ub_seed=%d outside {0,1,2}", sp->ub_seed);
    if (!out->topk_d || !out->topk_i)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "topk outputs are NULL");
    if ((out->probe_cids || out->probe_dqcs) && out->probe_ld < nprobe)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "probe_ld=%d < nprobe=%d", out->probe_ld, nprobe);
    const bool cascade = mode == TRIDENT_MODE_CASCADE;
    // modes 0 / 1: SQ8 reconstruction distance in the rotated space
    const bool hat = mode == TRIDENT_MODE_SQ8 || mode == TRIDENT_MODE_SQ8_RERANK;
    if ((cascade || hat) && (rc = validate_cascade_index(ix, hat))) return rc;
    if (sp->use_l1 && cascade && !ix->tile_r_minmax)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "use_l1 needs tile_r_minmax");
    if (mode == TRIDENT_MODE_TRIBASE && !ix->r_vec_sorted)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "mode 11 needs r_vec_sorted");
    // Mode 0 with a rerank: pass p keeps k_p entries per pair (reference :1439-1443, K_LOC :576)
    const int64_t eff_rr = mode == TRIDENT_MODE_SQ8_RERANK && sp->rerank_m > 0
                               ? std::max<int64_t>(sp->rerank_m, K) : 0;
    const int64_t M_rr = rerank_len(mode, K, sp->rerank_m);
    int64_t k_p1 = K, k_p2 = K;
    if (eff_rr > 0) {
        k_p1 = std::min<int64_t>(eff_rr, 128);
        k_p2 = std::min<int64_t>(
            eff_rr, std::max<int64_t>(K, std::max<int64_t>(16, (eff_rr + nprobe - 1) / nprobe + 8)));
        k_p2 = std::min<int64_t>(k_p2, 200);
    }
    const int64_t K_list = merged_list_len(mode, K, sp->rerank_m);
    if (B == 0) return TRIDENT_OK;
    if (!xq) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "xq is NULL");

    Workspace w = carve(ix, workspace, B, nprobe, K_list);
    if (!workspace || workspace_bytes < w.bytes)
        return fail(TRIDENT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu < %zu bytes", workspace_bytes,
                    w.bytes);
    hipStream_t st = static_cast<hipStream_t>(stream);

    int p_init =
        sp->p_init >= 0 ? sp->p_init : trident_p_init_rule(mode, B, K, nprobe, sp->rerank_m);
    if (mode == TRIDENT_MODE_CM_EXACT) p_init = 0;
    if (p_init > nprobe) p_init = nprobe;

    // Probes always land in the workspace (row stride nprobe); the caller's buffers, when
    // given, receive a mirror copy from the same kernel.
    int32_t* pc = w.probe_cids;
    float* pd = w.probe_dqcs;
    const int ld = nprobe;
    auto mark = [&](int ev) -> int {
        if (!out->events || ev >= out->n_events || !out->events[ev]) return TRIDENT_OK;
        hipError_t e = hipEventRecord(static_cast<hipEvent_t>(out->events[ev]), st);
        return e == hipSuccess ? TRIDENT_OK
                               : fail(TRIDENT_ERR_HIP, "hipEventRecord: %s", hipGetErrorString(e));
    };
    if ((rc = mark(TRIDENT_EV_START))) return rc;
    if ((rc = run_front_end(ix, xq, B, nprobe, cascade || hat, w, out->probe_cids,
                            out->probe_dqcs, out->probe_ld, st)))
        return rc;
    if ((rc = mark(TRIDENT_EV_PROBED))) return rc;

    // where the base lives: mapped host memory (out of core) changes the refine and, with
    // residual codes, the seeding; the PCIe telemetry counts rows read from there
    bool xb_host = false;
    {
        hipPointerAttribute_t pa;
        xb_host = hipPointerGetAttributes(&pa, ix->xb_sorted) == hipSuccess &&
                  pa.type == hipMemoryTypeHost;
        (void)hipGetLastError();  // an unregistered pointer is not an error here
    }
    int route = TRIDENT_ROUTE_PAIR;
    if (cascade && (rc = choose_route(ix, sp, B, K, nprobe, &route))) return rc;
    bool cm = false;
    if (mode == TRIDENT_MODE_CM_EXACT &&
        (rc = choose_cm_route(ix, sp, B, K, nprobe, xb_host, &cm)))
        return rc;
    // both batched routes group the pairs cluster-major in one array
    const bool batched = route == TRIDENT_ROUTE_BATCHED || cm;
    // the matrix-core mode 10 first scans each query's nearest probe (p_init of them when the
    // caller sets it) for thresholds only, so that its other probes, scanned together, start
    // from a threshold instead of +inf
    if (cm) p_init = sp->p_init >= 0 ? std::min(sp->p_init, nprobe) : (nprobe > 1 ? 1 : 0);
    const int64_t M1 = (int64_t)B * p_init, M2 = (int64_t)B * (nprobe - p_init);
    // per-pair route: the two passes' pairs in consecutive arrays; batched: one cluster-major
    // array (group_pairs)
    int32_t *p1c = w.pair_cids, *p1q = w.pair_qids;
    float* p1d = w.pair_dqcs;
    int32_t *p2c = batched ? p1c : w.pair_cids + M1, *p2q = batched ? p1q : w.pair_qids + M1;
    float* p2d = batched ? p1d : w.pair_dqcs + M1;
    if ((rc = group_pairs(pc, pd, ld, B, nprobe, p_init, ix->nlist, w.counts, w.seg_off, w.cursor,
                          p1c, p1q, pd ? p1d : nullptr, p2c, p2q, pd ? p2d : nullptr, batched, w.blk_tot,
                          w.pair_rank, st)))
        return rc;
    if ((rc = mark(TRIDENT_EV_GROUPED))) return rc;

    const int KP = list_kp(K_list);
    const int64_t cap = cand_cap(nprobe, K_list, ix->D_pad, ix->fine_codes && ix->fine_qp);
    if (out->stats) {
        if ((rc = fill(reinterpret_cast<int32_t*>(out->stats), 0, 8, st))) return rc;
        if ((rc = fill(reinterpret_cast<int32_t*>(w.stat_slots), 0, 2 * 4 * kStatSlots, st))) return rc;
    }
    unsigned long long* host_rows =
        out->host_rows && xb_host ? reinterpret_cast<unsigned long long*>(out->host_rows) : nullptr;
    if (out->host_rows && (rc = fill(reinterpret_cast<int32_t*>(out->host_rows), 0, 2, st))) return rc;
    if (out->host_rows_seed &&
        (rc = fill(reinterpret_cast<int32_t*>(out->host_rows_seed), 0, 2, st)))
        return rc;
    // at the end of the seeding pass: the rows it read from host memory so far
    auto seed_rows = [&]() -> int {
        if (!out->host_rows_seed || !host_rows) return TRIDENT_OK;
        copy_u64_kernel<<<1, 64, 0, st>>>(host_rows,
                                          reinterpret_cast<unsigned long long*>(out->host_rows_seed));
        return check_launch("copy_u64_kernel");
    };
    ScanArgs a = make_scan_args(ix, w, K, cap, cascade ? sp->use_l1 : 0,
                                out->stats ? w.stat_slots : nullptr);
    a.r_vec = ix->r_vec_sorted;
    a.host_rows = host_rows;
    MergeArgs m{};
    m.host_rows = host_rows;
    m.B = B;
    m.K = (int)K_list;
    m.hat = hat ? 1 : 0;
    m.cap = (int)cap;
    m.cand_key = w.cand_key;
    m.cand_id = w.cand_id;
    m.cand_cnt = w.cand_cnt;
    m.list_key = w.list_key;
    m.list_id = w.list_id;
    m.tau64 = w.tau64;

    if (cm) {
        // mode 10 on the matrix cores: one pass over every probe; the listed rows carry (lb, ub)
        // keys, tau = the K-th smallest listed ub, and the refine reads rows with lb <= tau only
        BatchArgs b{};
        b.vec_off = ix->cluster_vec_off;
        b.xb = ix->xb_sorted;
        b.xb8 = ix->xb_sorted_u8;
        b.orig_ids = ix->orig_ids_sorted;
        b.D = ix->D;
        b.D_pad = ix->D_pad;
        b.xq = xq;
        b.qerr = w.qerr;
        b.tau = w.tau64;
        b.B = B;
        b.xb_host = xb_host ? 1 : 0;
        b.host_rows = host_rows;
        b.cand_key = w.cand_key;
        b.cand_id = w.cand_id;
        b.cand_cnt = w.cand_cnt;
        b.cap = (int)cap;
        b.K = K;
        b.stats = out->stats ? w.stat_slots : nullptr;
        b.units = w.units;
        b.unit_off = w.unit_off;
        b.max_units = (int)w.max_units;
        b.pair_qid = w.pair_qids;
        b.pair_cid = w.pair_cids;
        b.seg = w.seg_off;
        b.M = (int)(M1 + M2);
        b.nlist = ix->nlist;
        b.unit_q = kUnitQWide;
        b.ub_cnt = w.ub_cnt;
        b.ub_best = w.ub_best;
        b.seed_cnt = w.seed_cnt;
        b.qep = w.qep;
        b.fine_mode = 1;  // the candidate keys hold (lb, ub): the refine skips lb > tau
        // per-query state (tau, counts, thresholds) and the work counters
        aux_bounds_kernel<<<(unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock), kBlock, 0,
                            st>>>(b, 0, B, w.cbound, w.qep, w.unit_ctr);
        if ((rc = check_launch("aux_bounds_kernel"))) return rc;
        {
            const int nblk = (2 * ix->nlist + kBlock - 1) / kBlock;
            unit_scan_local_kernel<<<nblk, kBlock, 0, st>>>(w.seg_off, ix->cluster_vec_off,
                                                            ix->nlist, b.unit_q, 0,
                                                            seed_slice_count(K, false, false),
                                                            kSplitVec, kSplitVec, w.unit_off, w.grp_off,
                                                            w.blk_tot);
            if ((rc = check_launch("unit_scan_local_kernel"))) return rc;
            unit_scan_carry_kernel<<<nblk, kBlock, 0, st>>>(ix->nlist, w.blk_tot, nblk,
                                                            w.unit_off, w.grp_off);
            if ((rc = check_launch("unit_scan_carry_kernel"))) return rc;
        }
        unit_fill_kernel<<<(unsigned)std::min<int64_t>((w.max_units + 255) / 256, 2048), 256, 0,
                           st>>>(w.seg_off, ix->cluster_vec_off, ix->nlist, b.unit_q, 0,
                                 kSplitVec, kSplitVec, w.unit_off, w.units, (int)w.max_units, w.grp_off,
                                 w.groups, (int)w.max_groups);
        if ((rc = check_launch("unit_fill_kernel"))) return rc;
        const unsigned qg = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
        if (M1 > 0) {
            // warm-up over the first probes: for K <= 16 the scan's own thresholds (the K-th
            // smallest of 16 column minima), nothing listed; past 16 every row is listed and
            // cm_seed_kernel takes the K-th smallest listed ub, then empties the lists
            b.cm_emit = K > 16 ? 1 : 0;
            b.unit_beg = 0;
            b.unit_end = ix->nlist;
            b.ctr = w.unit_ctr;
            if ((rc = launch_cm(b, st))) return rc;
            if (K > 16) {
                if (K <= 64) cm_seed_kernel<64><<<qg, kBlock, 0, st>>>(b, B);
                else cm_seed_kernel<128><<<qg, kBlock, 0, st>>>(b, B);
                if ((rc = check_launch("cm_seed_kernel"))) return rc;
            }
        }
        if ((rc = mark(TRIDENT_EV_P1_SCAN))) return rc;
        if ((rc = mark(TRIDENT_EV_P1_MERGE))) return rc;
        // every probe (the first ones again: the warm-up listed nothing)
        b.cm_emit = 1;
        b.unit_beg = ix->nlist;
        b.unit_end = 2 * ix->nlist;
        b.ctr = w.unit_ctr + 8 * kCtrStride;
        if ((rc = launch_cm(b, st))) return rc;
        if ((rc = mark(TRIDENT_EV_P2_SCAN))) return rc;
        if (K <= 64) fine_tau_kernel<64><<<qg, kBlock, 0, st>>>(b, B);
        else fine_tau_kernel<128><<<qg, kBlock, 0, st>>>(b, B);
        if ((rc = check_launch("fine_tau_kernel"))) return rc;
        const dim3 rgrid(qg, (unsigned)std::min<int64_t>((cap + kWave - 1) / kWave, 16));
        if (ix->D <= 256) {
            if (xb_host) refine_survivors_kernel<true, 256><<<rgrid, kBlock, 0, st>>>(b, B);
            else refine_survivors_kernel<false, 256><<<rgrid, kBlock, 0, st>>>(b, B);
        } else {
            if (xb_host) refine_survivors_kernel<true, 1024><<<rgrid, kBlock, 0, st>>>(b, B);
            else refine_survivors_kernel<false, 1024><<<rgrid, kBlock, 0, st>>>(b, B);
        }
        if ((rc = check_launch("refine_survivors_kernel"))) return rc;
        m.use_prev = 0;
        m.tau_sq_out = out->tau_sq;
        m.out_d = out->topk_d;
        m.out_i = out->topk_i;
        m.probe_cids = w.probe_cids;
        m.nprobe = nprobe;
        m.vec_off = ix->cluster_vec_off;
        m.xb = ix->xb_sorted;
        m.xq64 = w.xq64;
        m.tile_oids = ix->tile_orig_ids;
        m.tile_off = ix->cluster_tile_off;
        m.T = ix->tile_size;
        m.D = ix->D;
        if ((rc = launch_merge(m, KP, st))) return rc;
        if ((rc = mark(TRIDENT_EV_END))) return rc;
        if (out->stats) {
            stats_fold_kernel<<<1, 64, 0, st>>>(w.stat_slots, out->stats);
            if ((rc = check_launch("stats_fold_kernel"))) return rc;
        }
        return TRIDENT_OK;
    }

    if (batched) {
        BatchArgs b{};
        b.cells = reinterpret_cast<const uint4*>(ix->sq8_cells);
        b.tile_oids = ix->tile_orig_ids;
        b.tile_off = ix->cluster_tile_off;
        b.vec_off = ix->cluster_vec_off;
        b.xb = ix->xb_sorted;
        b.xb8 = ix->xb_sorted_u8;
        b.vmin = ix->vmin;
        b.delta = ix->delta;
        b.eps = ix->eps_dim;
        b.orig_ids = ix->orig_ids_sorted;
        b.vec_Ar = reinterpret_cast<const float2*>(ix->vec_Ar);
        b.vec_cn = ix->vec_cn;
        b.D = ix->D;
        b.D_pad = ix->D_pad;
        b.T = ix->tile_size;
        b.per_cluster = ix->per_cluster_sq8;
        b.xq = xq;
        b.xrot64 = w.xrot64;
        b.xrot32 = w.xrot32;
        b.qerr = w.qerr;
        b.tau = w.tau64;
        b.tau_sq_out = nullptr;
        b.B = B;
        b.xb_host = xb_host ? 1 : 0;
        b.host_rows = host_rows;
        b.cand_key = w.cand_key;
        b.cand_id = w.cand_id;
        b.cand_cnt = w.cand_cnt;
        b.cap = (int)cap;
        b.K = K;
        b.stats = out->stats ? w.stat_slots : nullptr;
        b.use_l1 = sp->use_l1 ? 1 : 0;
        b.tile_rmm = ix->tile_r_minmax;
        b.pair_dqc = w.pair_dqcs;
        b.rot_sq_min = ix->rot_sq_min;
        b.rot_sq_max = ix->rot_sq_max;
        b.sum_rel = sum_rel_of(ix->D_pad);
        // fine level: used when the rows live across PCIe (the seeds' and survivors' bounds
        // then come from HBM, and only rows that can still enter the top-K are read)
        b.fine_codes = ix->fine_codes;
        b.fine_qp = ix->fine_qp;
        b.fine_mode = ix->fine_codes && ix->fine_qp && b.xb_host ? 1 : 0;
        b.units = w.units;
        b.unit_off = w.unit_off;
        b.max_units = (int)w.max_units;
        b.pair_qid = w.pair_qids;
        b.pair_cid = w.pair_cids;
        b.seg = w.seg_off;
        b.M = (int)(M1 + M2);
        b.unit_q = lb_unit_q(ix->D_pad);
        b.DP = (int)plane_bytes(ix->D_pad);
        b.pw = w.pw;
        b.prec = w.prec;
        b.lbr = w.lbr;
        b.lbk = w.lbk;
        // index-constant per-cluster bounds: the view's table when it has one
        b.cbound = ix->cluster_bounds ? ix->cluster_bounds : w.cbound;
        b.qep = w.qep;
        b.ub_list = w.ub_list;
        b.ub_cnt = w.ub_cnt;
        b.ub_best = w.ub_best;
        b.seed_cnt = w.seed_cnt;
        b.ub_cap = (int)w.ub_cap;
        b.nlist = ix->nlist;
        b.groups = w.groups;
        b.grp_off = w.grp_off;
        b.max_groups = (int)w.max_groups;
        const int ncl = ix->cluster_bounds ? 0 : ix->nlist;
        aux_bounds_kernel<<<(unsigned)((ncl + B + kWavesPerBlock - 1) / kWavesPerBlock), kBlock,
                            0, st>>>(b, ncl, B, w.cbound, w.qep, w.unit_ctr);
        if ((rc = check_launch("aux_bounds_kernel"))) return rc;
        // TRIDENT_UB_SEED 2 seeds from every probe, 0 and 1 from the first p_init
        const int seed_all = sp->ub_seed == 2 ? 1 : 0;
        const int split_vec = ix->D_pad <= 256 ? kSplitVecNarrow : kSplitVec;
        const int split_vec_b =
            ix->D_pad <= 256 && (int64_t)ix->N >= (int64_t)kLongSliceRows * ix->nlist ? 2 * kSplitVecNarrow
                                                                                  : split_vec;
        const int seed_sl = seed_slice_count(K, xb_host, b.fine_mode != 0);
        // seeding slices: split_vec rows, or the index's seed_rows (at least 512, so that no
        // slice is empty) when its rows within a cluster put the best seeds first
        const int split_vec_a =
            ix->seed_rows > 0 ? std::max(512, std::min(split_vec, (int)ix->seed_rows)) : split_vec;
        {
            const int nblk = (2 * ix->nlist + kBlock - 1) / kBlock;  // <= kBlock (kMaxBatchedNlist)
            unit_scan_local_kernel<<<nblk, kBlock, 0, st>>>(w.seg_off, ix->cluster_vec_off,
                                                            ix->nlist, b.unit_q, seed_all, seed_sl,
                                                            split_vec_a, split_vec_b, w.unit_off, w.grp_off,
                                                            w.blk_tot);
            if ((rc = check_launch("unit_scan_local_kernel"))) return rc;
            unit_scan_carry_kernel<<<nblk, kBlock, 0, st>>>(ix->nlist, w.blk_tot, nblk,
                                                            w.unit_off, w.grp_off);
            if ((rc = check_launch("unit_scan_carry_kernel"))) return rc;
        }
        unit_fill_kernel<<<(unsigned)std::min<int64_t>((w.max_units + 255) / 256, 2048), 256, 0,
                           st>>>(w.seg_off, ix->cluster_vec_off, ix->nlist, b.unit_q, seed_all,
                                 split_vec_a, split_vec_b, w.unit_off, w.units, (int)w.max_units, w.grp_off,
                                 w.groups, (int)w.max_groups);
        if ((rc = check_launch("unit_fill_kernel"))) return rc;
        if ((rc = launch_pair_prep(b, st))) return rc;
        if (M1 > 0 || seed_all) {
            // pass A: per-query upper bounds from the seeding probes, then the exact distances of
            // each query's K best-bound rows (the seeds) set the threshold
            b.unit_beg = 0;
            b.unit_end = ix->nlist;
            b.ctr = w.unit_ctr;
            if ((rc = launch_batch<true>(b, st))) return rc;
            const unsigned kg = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
            if (K <= 64) {
                if (ix->D <= 256) ub_kth_kernel<64, 256><<<kg, kBlock, 0, st>>>(b);
                else ub_kth_kernel<64, 1024><<<kg, kBlock, 0, st>>>(b);
            } else {
                if (ix->D <= 256) ub_kth_kernel<128, 256><<<kg, kBlock, 0, st>>>(b);
                else ub_kth_kernel<128, 1024><<<kg, kBlock, 0, st>>>(b);
            }
            if ((rc = check_launch("ub_kth_kernel"))) return rc;
        }
        if ((rc = mark(TRIDENT_EV_P1_SCAN))) return rc;
        // the lower-bound constants follow from tau (part of the seeding pass's merge stage);
        // the same launch hands the caller its float32 copy of tau
        b.tau_sq_out = out->tau_sq;
        lb_prep_kernel<<<(unsigned)std::max<int64_t>(
                             (w.max_groups + kBlock / kGroupQ - 1) / (kBlock / kGroupQ), 1),
                         kBlock, 0, st>>>(b);
        if ((rc = check_launch("lb_prep_kernel"))) return rc;
        if ((rc = seed_rows())) return rc;
        if ((rc = mark(TRIDENT_EV_P1_MERGE))) return rc;
        // pass B over every probe: lower bound, exact refine, append <= tau
        b.unit_beg = ix->nlist;
        b.unit_end = 2 * ix->nlist;
        b.ctr = w.unit_ctr + 8 * kCtrStride;
        if ((rc = launch_batch<false>(b, st))) return rc;
        if ((rc = mark(TRIDENT_EV_P2_SCAN))) return rc;
        if (b.fine_mode) {
            const unsigned qg = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
            const dim3 fgrid(qg, (unsigned)std::min<int64_t>((cap + kWave - 1) / kWave, 16));
            if (ix->D <= 256) fine_filter_kernel<256><<<fgrid, kBlock, 0, st>>>(b, B);
            else fine_filter_kernel<1024><<<fgrid, kBlock, 0, st>>>(b, B);
            if ((rc = check_launch("fine_filter_kernel"))) return rc;
            if (K <= 64) fine_tau_kernel<64><<<qg, kBlock, 0, st>>>(b, B);
            else fine_tau_kernel<128><<<qg, kBlock, 0, st>>>(b, B);
            if ((rc = check_launch("fine_tau_kernel"))) return rc;
        }
        // one wave per (query, 64-slot chunk of its list): a query with many survivors spreads
        // over many waves
        // the chunk dimension stops at 16: waves loop over further chunks
        const dim3 rgrid((unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock),
                         (unsigned)std::min<int64_t>((cap + kWave - 1) / kWave, 16));
        if (ix->D <= 256) {
            if (b.xb_host)
                refine_survivors_kernel<true, 256><<<rgrid, kBlock, 0, st>>>(b, B);
            else
                refine_survivors_kernel<false, 256><<<rgrid, kBlock, 0, st>>>(b, B);
        } else {
            if (b.xb_host)
                refine_survivors_kernel<true, 1024><<<rgrid, kBlock, 0, st>>>(b, B);
            else
                refine_survivors_kernel<false, 1024><<<rgrid, kBlock, 0, st>>>(b, B);
        }
        if ((rc = check_launch("refine_survivors_kernel"))) return rc;
        m.use_prev = 0;
        m.out_d = out->topk_d;
        m.out_i = out->topk_i;
        m.probe_cids = w.probe_cids;
        m.nprobe = nprobe;
        m.vec_off = ix->cluster_vec_off;
        m.xb = ix->xb_sorted;
        m.xq64 = w.xq64;
        m.tile_oids = ix->tile_orig_ids;
        m.tile_off = ix->cluster_tile_off;
        m.T = ix->tile_size;
        m.D = ix->D;
        // an overflowed list is rescanned through the SQ8 bounds (rows near the top-K only)
        m.ovf_bounds = 1;
        m.cells = reinterpret_cast<const uint4*>(ix->sq8_cells);
        m.vmin = ix->vmin;
        m.delta = ix->delta;
        m.eps = ix->eps_dim;
        m.per_cluster = ix->per_cluster_sq8;
        m.D_pad = ix->D_pad;
        m.xrot64 = w.xrot64;
        m.qerr = w.qerr;
        m.lb_scale = a.lb_scale;
        m.ub_scale = a.ub_scale;
        // up to ovf_max overflowed lists are rescanned in parallel, one wave per (query, probe);
        // without an overflow the launches find no slot and end at once
        m.ovf_par = KP <= 128 ? 1 : 0;
        if (m.ovf_par) {
            m.ovf_max = (int)w.ovf_max;
            m.ovf_n = w.ovf_n;
            m.ovf_q = w.ovf_q;
            m.ovf_slot = w.ovf_slot;
            m.ovf_t = w.ovf_t;
            m.ovf_key = w.ovf_key;
            m.ovf_id = w.ovf_id;
            if ((rc = fill(w.ovf_n, 0, 1, st))) return rc;
            ovf_collect_kernel<<<(unsigned)((B + 255) / 256), 256, 0, st>>>(m);
            if ((rc = check_launch("ovf_collect_kernel"))) return rc;
            const size_t odyn = (size_t)kWavesPerBlock * 3 * ix->D_pad * sizeof(float);
            const unsigned og = (unsigned)std::min<int64_t>(
                (w.ovf_max * nprobe + kWavesPerBlock - 1) / kWavesPerBlock, 2048);
            const unsigned kg = (unsigned)((w.ovf_max + kWavesPerBlock - 1) / kWavesPerBlock);
            if (KP == 64) {
                ovf_scan_kernel<64, true><<<og, kBlock, odyn, st>>>(m);
                ovf_kth_kernel<64><<<kg, kBlock, 0, st>>>(m);
                ovf_scan_kernel<64, false><<<og, kBlock, odyn, st>>>(m);
            } else {
                ovf_scan_kernel<128, true><<<og, kBlock, odyn, st>>>(m);
                ovf_kth_kernel<128><<<kg, kBlock, 0, st>>>(m);
                ovf_scan_kernel<128, false><<<og, kBlock, odyn, st>>>(m);
            }
            if ((rc = check_launch("ovf_scan_kernel"))) return rc;
        }
        if ((rc = launch_merge(m, KP, st))) return rc;
        if ((rc = mark(TRIDENT_EV_END))) return rc;
        if (out->stats) {
            stats_fold_kernel<<<1, 64, 0, st>>>(w.stat_slots, out->stats);
            if ((rc = check_launch("stats_fold_kernel"))) return rc;
        }
        return TRIDENT_OK;
    }

    // the scan kind of each pass
    const int kind1 = cascade ? (sp->ub_seed != 0 ? kScanCascadeUb : kScanCascade)
                      : hat   ? kScanHat
                      : mode == TRIDENT_MODE_TRIBASE ? kScanTribase
                                                     : kScanExact;
    const int kind2 = cascade ? (sp->ub_seed == 2 || (sp->ub_seed == 1 && M1 == 0) ? kScanCascadeUb
                                                                                   : kScanCascade)
                              : kind1;
    // mode 0 with a rerank: the merges only build the top-M list; rerank_kernel writes the outputs
    const bool rerank = eff_rr > 0;
    if (M1 > 0) {
        if ((rc = fill(w.cand_cnt, 0, B, st))) return rc;
        a.pair_cid = p1c;
        a.pair_qid = p1q;
        a.pair_dqc = pd ? p1d : nullptr;
        a.M = (int)M1;
        a.K = (int)k_p1;
        a.tau_in = nullptr;
        if ((rc = dispatch_scan(a, kind1, st))) return rc;
        if ((rc = mark(TRIDENT_EV_P1_SCAN))) return rc;
        m.use_prev = 0;
        m.tau_sq_out = out->tau_sq;
        const bool last = M2 == 0 && !rerank;
        m.out_d = last ? out->topk_d : nullptr;
        m.out_i = last ? out->topk_i : nullptr;
        if ((rc = launch_merge(m, KP, st))) return rc;
    } else if ((rc = mark(TRIDENT_EV_P1_SCAN))) {
        return rc;
    }
    if ((rc = seed_rows())) return rc;
    if ((rc = mark(TRIDENT_EV_P1_MERGE))) return rc;
    if (M2 > 0) {
        if ((rc = fill(w.cand_cnt, 0, B, st))) return rc;
        a.pair_cid = p2c;
        a.pair_qid = p2q;
        a.pair_dqc = pd ? p2d : nullptr;
        a.M = (int)M2;
        a.K = (int)k_p2;
        // acc_hat lists take no threshold: tau64 bounds exact distances only
        a.tau_in = M1 > 0 && !hat ? w.tau64 : nullptr;
        if ((rc = dispatch_scan(a, kind2, st))) return rc;
        if ((rc = mark(TRIDENT_EV_P2_SCAN))) return rc;
        m.use_prev = M1 > 0 ? 1 : 0;
        m.tau_sq_out = M1 > 0 ? nullptr : out->tau_sq;
        m.out_d = rerank ? nullptr : out->topk_d;
        m.out_i = rerank ? nullptr : out->topk_i;
        if ((rc = launch_merge(m, KP, st))) return rc;
    } else if ((rc = mark(TRIDENT_EV_P2_SCAN))) {
        return rc;
    }
    if (rerank) {
        RerankArgs r{};
        r.B = B;
        r.K = K;
        r.M = (int)M_rr;
        r.list_key = w.list_key;
        r.list_id = w.list_id;
        r.KP = KP;
        r.xb = ix->xb_sorted;
        r.xq64 = w.xq64;
        r.D = ix->D;
        r.out_d = out->topk_d;
        r.out_i = out->topk_i;
        r.host_rows = host_rows;
        if ((rc = K <= 64 ? launch_rerank<64>(r, st) : launch_rerank<128>(r, st))) return rc;
    }
    if ((rc = mark(TRIDENT_EV_END))) return rc;
    if (out->stats) {
        stats_fold_kernel<<<1, 64, 0, st>>>(w.stat_slots, out->stats);
        if ((rc = check_launch("stats_fold_kernel"))) return rc;
    }
    return TRIDENT_OK;
}

int trident_search_noalloc(const TridentIndexView* ix, const TridentSearchParams* sp,
                           const float* xq, const TridentSearchOutputs* out, void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if (!sp || !out) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "params/outputs are NULL");
    if (sp->B < 0 || sp->K < 1 || sp->nprobe < 1)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad sizes B=%d K=%d nprobe=%d", sp->B, sp->K,
                    sp->nprobe);
    // the size check comes before any HIP call, so an oversized request fails without touching
    // the device
    const size_t need =
        carve(ix, nullptr, sp->B, sp->nprobe, merged_list_len(sp->mode, sp->K, sp->rerank_m)).bytes;
    if (need > (size_t)TRIDENT_NOALLOC_SCRATCH_BYTES)
        return fail(TRIDENT_ERR_WORKSPACE_TOO_SMALL,
                    "trident_search_noalloc: B=%d nprobe=%d K=%d needs %zu bytes of scratch, more "
                    "than the fixed %zu (use trident_search with a caller-owned workspace)",
                    sp->B, sp->nprobe, sp->K, need, (size_t)TRIDENT_NOALLOC_SCRATCH_BYTES);
    if (stream) {
        int sdev = -1, cur = -1;
        hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
        if (e == hipSuccess) e = hipGetDevice(&cur);
        if (e != hipSuccess)
            return fail(TRIDENT_ERR_HIP, "stream device: %s", hipGetErrorString(e));
        if (sdev != cur)
            return fail(TRIDENT_ERR_INVALID_ARGUMENT,
                        "trident_search_noalloc: the stream is on device %d, make it current (current "
                        "device %d)", sdev, cur);
    }
    void* ws = nullptr;
    if ((rc = scratch_of_current_device(&ws))) return rc;
    return trident_search(ix, sp, xq, ws, (size_t)TRIDENT_NOALLOC_SCRATCH_BYTES, out, stream);
}

int trident_sq8_bounds(const TridentIndexView* ix, const float* xq, int32_t B,
                       const int32_t* qids, const int32_t* cids, const int64_t* spos, int32_t n,
                       void* workspace, size_t workspace_bytes, double* lb, double* ub,
                       void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if ((rc = validate_cascade_index(ix))) return rc;
    if (B < 1 || n < 0 || !xq || !qids || !cids || !spos || !lb || !ub)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad sq8_bounds arguments");
    Workspace w = carve(ix, workspace, B, 1, 1);
    if (!workspace || workspace_bytes < w.bytes)
        return fail(TRIDENT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu < %zu bytes", workspace_bytes,
                    w.bytes);
    if (n == 0) return TRIDENT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int ldw = ix->nlist + ix->D_pad;
    const int cols = std::max(ix->D, ix->D_pad);
    prep_queries_kernel<<<dim3((cols + 127) / 128, (B + 4 * kPrepQB - 1) / (4 * kPrepQB)),
                          dim3(64, 4), 0, st>>>(
        xq, B, ix->D, ix->D_pad, ix->W_combined, ldw, ix->nlist, ix->b_combined, w.xq64,
        w.xrot64, w.xrot32, w.qerr, 1);
    if ((rc = check_launch("prep_queries_kernel"))) return rc;
    ScanArgs a = make_scan_args(ix, w, 1, 1, 0, nullptr);
    sq8_bounds_kernel<<<(n + 255) / 256, 256, 0, st>>>(a, qids, cids, spos, n, lb, ub);
    return check_launch("sq8_bounds_kernel");
}

int trident_cluster_bounds(const TridentIndexView* ix, double* cluster_bounds, void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if (!ix->vec_Ar || !ix->delta || !ix->eps_dim || !cluster_bounds)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "cluster_bounds needs vec_Ar, delta, eps_dim");
    BatchArgs b{};
    b.D_pad = ix->D_pad;
    b.per_cluster = ix->per_cluster_sq8;
    b.delta = ix->delta;
    b.eps = ix->eps_dim;
    b.vec_off = ix->cluster_vec_off;
    b.vec_Ar = reinterpret_cast<const float2*>(ix->vec_Ar);
    aux_bounds_kernel<<<(unsigned)((ix->nlist + kWavesPerBlock - 1) / kWavesPerBlock), kBlock, 0,
                        static_cast<hipStream_t>(stream)>>>(b, ix->nlist, 0, cluster_bounds,
                                                            nullptr, nullptr);
    return check_launch("aux_bounds_kernel");
}

int trident_fine_bounds(const TridentIndexView* ix, const float* xq, int32_t B,
                       const int32_t* qids, const int64_t* spos, int32_t n, void* workspace,
                       size_t workspace_bytes, double* lb, double* ub, void* stream) {
    int rc = validate_index(ix);
    if (rc) return rc;
    if (!ix->fine_codes || !ix->fine_qp)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "fine_bounds needs fine_codes and fine_qp");
    if (B < 1 || n < 0 || !xq || !qids || !spos || !lb || !ub)
        return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad fine_bounds arguments");
    Workspace w = carve(ix, workspace, B, 1, 1);
    if (!workspace || workspace_bytes < w.bytes)
        return fail(TRIDENT_ERR_WORKSPACE_TOO_SMALL, "workspace %zu < %zu bytes", workspace_bytes,
                    w.bytes);
    if (n == 0) return TRIDENT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int ldw = ix->nlist + ix->D_pad;
    const int cols = std::max(ix->D, ix->D_pad);
    prep_queries_kernel<<<dim3((cols + 127) / 128, (B + 4 * kPrepQB - 1) / (4 * kPrepQB)),
                          dim3(64, 4), 0, st>>>(
        xq, B, ix->D, ix->D_pad, ix->W_combined, ldw, ix->nlist, ix->b_combined, w.xq64,
        w.xrot64, w.xrot32, w.qerr, 1);
    if ((rc = check_launch("prep_queries_kernel"))) return rc;
    BatchArgs b{};
    b.D = ix->D;
    b.D_pad = ix->D_pad;
    b.xrot64 = w.xrot64;
    b.qerr = w.qerr;
    b.rot_sq_min = ix->rot_sq_min;
    b.rot_sq_max = ix->rot_sq_max;
    b.fine_codes = ix->fine_codes;
    b.fine_qp = ix->fine_qp;
    fine_bounds_kernel<<<(n + 255) / 256, 256, 0, st>>>(b, qids, spos, n, lb, ub);
    return check_launch("fine_bounds_kernel");
}

int trident_event_create(void** event) {
    if (!event) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "NULL event pointer");
    hipEvent_t e;
    hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) return fail(TRIDENT_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(r));
    *event = e;
    return TRIDENT_OK;
}

int trident_event_destroy(void* event) {
    if (!event) return TRIDENT_OK;
    hipError_t r = hipEventDestroy(static_cast<hipEvent_t>(event));
    return r == hipSuccess ? TRIDENT_OK
                           : fail(TRIDENT_ERR_HIP, "hipEventDestroy: %s", hipGetErrorString(r));
}

int trident_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (!start || !stop || !ms) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "NULL event argument");
    hipError_t r = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
    return r == hipSuccess ? TRIDENT_OK
                           : fail(TRIDENT_ERR_HIP, "hipEventElapsedTime: %s", hipGetErrorString(r));
}

int trident_host_alloc_mapped(size_t bytes, void** host_ptr) {
    if (!host_ptr || bytes == 0) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "bad host alloc args");
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocPortable);
    if (e != hipSuccess)
        return fail(TRIDENT_ERR_OUT_OF_MEMORY, "hipHostMalloc(%zu): %s", bytes,
                    hipGetErrorString(e));
    *host_ptr = p;
    return TRIDENT_OK;
}

int trident_host_free(void* host_ptr) {
    if (!host_ptr) return TRIDENT_OK;
    hipError_t e = hipHostFree(host_ptr);
    if (e != hipSuccess) return fail(TRIDENT_ERR_HIP, "hipHostFree: %s", hipGetErrorString(e));
    return TRIDENT_OK;
}

int trident_host_device_pointer(void* host_ptr, void** device_ptr) {
    if (!host_ptr || !device_ptr) return fail(TRIDENT_ERR_INVALID_ARGUMENT, "NULL pointer");
    hipError_t e = hipHostGetDevicePointer(device_ptr, host_ptr, 0);
    if (e != hipSuccess)
        return fail(TRIDENT_ERR_HIP, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
    return TRIDENT_OK;
}

}  // extern "C"
