// Kernel declarations and argument blocks of the gfx950 lossless IVF query path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trident {

// Everything one per-pair scan launch reads; passed by value as the kernel argument.
struct ScanArgs {
    // index layout
    const uint32_t* sq8;        // [tiles, D4, T]
    const int32_t* tile_oids;   // [tiles, T]
    const float* tile_rmm;      // [tiles, 2] or null
    const int32_t* tile_off;    // [nlist + 1]
    const int32_t* vec_off;     // [nlist + 1]
    const float* xb;            // [N, D] sorted base (device or mapped host)
    const float* vmin;          // [nlist|1, D_pad]
    const float* delta;
    const float* eps;
    const int32_t* blk;         // [nb + 1]
    int D, D_pad, T, nb, per_cluster, use_l1;
    // queries
    const double* xq64;         // [B, D]
    const double* xrot64;       // [B, D_pad]
    const double* qerr;         // [B, D_pad]
    // pairs of this pass, grouped by cluster
    const int32_t* pair_cid;
    const int32_t* pair_qid;
    const float* pair_dqc;      // |q - c| per pair (use_l1, Tribase) or null
    const float* r_vec;         // [N] |x - c| in sorted order (Tribase) or null
    int M;
    // per-query threshold from the previous pass (float64), or null
    const double* tau_in;
    // per-query candidate lists
    uint64_t* cand_key;
    int32_t* cand_id;
    int32_t* cand_cnt;
    int cap, K;                 // K: entries kept (and emitted) per pair
    unsigned long long* stats;  // [4] or null
    unsigned long long* host_rows;  // [1] rows read from a host-mapped base, or null
    double lb_scale;            // tau -> float32 Stage Y threshold factor
    double ub_scale;            // Stage X sum -> float64 distance bound factor
};

struct MergeArgs {
    int B, K, cap;
    const uint64_t* cand_key;
    const int32_t* cand_id;
    const int32_t* cand_cnt;
    uint64_t* list_key;   // [B, KP] per-query running top list
    int32_t* list_id;
    int use_prev;
    // 1: keys are (acc_hat bits, original id) (kScanHat): out_d / tau_sq_out receive acc_hat,
    // out_i the original id, tau64 is set to +inf
    int hat;
    double* tau64;        // [B] K-th distance after this merge (+inf if fewer than K)
    float* out_d;         // [B, K] or null (final pass only)
    int64_t* out_i;
    float* tau_sq_out;    // [B] or null
    // Rescan of a query whose candidate list overflowed `cap` (only the batched routes append
    // without a per-pair cap): through the SQ8 bounds (ovf_bounds below), else every probed row
    // refined exactly (mode 10's matrix route, whose index carries no SQ8 codes).
    const int32_t* probe_cids;  // [B, nprobe] or null (no fallback needed)
    int nprobe;
    const int32_t* vec_off;
    const float* xb;
    const double* xq64;   // [B, D]
    const int32_t* tile_oids;
    const int32_t* tile_off;
    int T, D;
    unsigned long long* host_rows;  // [1] rows read by the rescan (host-mapped base), or null
    // Bounded rescan (ovf_bounds = 1, the batched cascade route): the overflowed query's probed
    // rows get their Stage X / Y bounds from the SQ8 code cells and the per-dim parameters
    // below; only rows whose lower bound passes the K-th smallest upper bound are read and
    // refined.
    int ovf_bounds;
    const uint4* cells;         // [tiles, T / V, D_pad / 16, V] (bytes c ^ 0x80)
    const float* vmin;
    const float* delta;
    const float* eps;
    int per_cluster, D_pad;
    const double* xrot64;       // [B, D_pad]
    const double* qerr;         // [B, D_pad]
    double lb_scale, ub_scale;  // as ScanArgs
    // Parallel bounded rescan (ovf_par = 1, with ovf_bounds): ovf_collect_kernel gives up to
    // ovf_max overflowed queries a slot; ovf_scan_kernel rescans them one wave per (slot, probe),
    // each keeping its cluster's K best in ovf_key / ovf_id [ovf_max, nprobe, KP] (upper bounds
    // first, reduced by ovf_kth_kernel to the slot's threshold ovf_t, then refined distances);
    // merge_kernel merges a slot's lists.  Overflowed queries past ovf_max take the serial rescan.
    int ovf_par, ovf_max;
    int32_t* ovf_n;       // [1] overflowed queries (may exceed ovf_max); zero before the collect
    int32_t* ovf_q;       // [ovf_max] the query of each slot
    int32_t* ovf_slot;    // [B] each query's slot, -1 for none
    double* ovf_t;        // [ovf_max]
    uint64_t* ovf_key;
    int32_t* ovf_id;
};

// Per-(query, cluster) pair scalars of the batched bound (threshold-independent part).
struct PairRec {
    double Qp;       // |q_rot - vmin|^2
    double err_q;    // 255 * sum |w - s w_int|  (bound on the weight quantisation error)
    double e_q;      // >= |q_rot(float64) - q_rot(exact)|
    double cW;       // 128 * sum w_int
    double c1;       // 2 s
    double a_max;    // >= A_x for every vector of the cluster
    double r_max;    // >= r_x for every vector of the cluster
    double acc_max;  // >= |sum c'_d w_int,d|
    double lo_max;   // 128 * sum |lo_d| >= |sum c'_d lo_d| (the lo plane's share of the sum)
    double lo_l2;    // >= sqrt(sum lo_d^2): |sum c'_d lo_d| <= |c'|_2 lo_l2 (Cauchy-Schwarz)
};

// Per-pair constants of the batched lower-bound scan (they depend on tau, so they are computed
// after the seeding pass).  int_ok, tqw and inv_c1w are shared by the pair's weight group.
struct LbRec {
    int32_t kq;        // integer test: acc + kq >= thr_x
    float c1f, c2f;    // float test: fma(c2f, r, P) <= fma(c1f, float(acc), H32)
    float H32;
    float tqw;         // the group's largest tq, rounded up
    float inv_c1w;     // 1 / c1 of the group (a power of two)
    int32_t int_ok;    // the group takes the integer test
    int32_t kq_pre;    // with the hi plane alone, acc_hi * 256 + kq_pre + lo_w * 256 * cn_x >= the
                       // sum: kq + lo_max and lo_w = 0 without row norms, else kq
    float lo_w;        // the group's largest lo_l2 / 256, rounded up (0 without row norms)
};

// Everything one cluster-batched scan launch reads (csrc/batch.hip).
struct BatchArgs {
    const uint4* cells;         // [tiles, T / V, D_pad / 16, V] 16-byte code cells (V-slot
                                // blocks contiguous, V = block_vectors), bytes c ^ 0x80
    const int32_t* tile_oids;
    const int32_t* tile_off;
    const int32_t* vec_off;
    const float* xb;
    const uint8_t* xb8;         // [N, D] the rows of xb as uint8 (exact), or null: read by the
                                // exact refines instead of xb (a quarter of the bytes)
    const float* vmin;
    const float* delta;
    const float* eps;           // per-dim |x_rot - x_hat| bound (bounds r_x for the f32 slack)
    const int32_t* orig_ids;    // [N] sorted position -> original id
    const float2* vec_Ar;       // [N] (A rounded down, r rounded up)
    const float* vec_cn;        // [N] >= |code - 128|_2 per row, or null
    int D, D_pad, T, per_cluster;
    const float* xq;            // [B, D] float32 queries
    const double* xrot64;       // [B, D_pad]
    const float* xrot32;        // [B, D_pad] xrot64 rounded to float32
    const double* qerr;         // [B, D_pad]
    const int4* units;          // work units {cid | cnt << 20, pair start, v_begin, v_end}
    const int32_t* unit_off;    // [2 * nlist + 1] unit offsets: seeding units of cluster c at
                                // [unit_off[c], unit_off[c + 1]), lower-bound units of cluster c
                                // at [unit_off[nlist + c], unit_off[nlist + c + 1])
    int unit_beg, unit_end;     // this launch covers units [unit_off[unit_beg], unit_off[unit_end])
    int max_units;
    int32_t* ctr;               // [8 * kCtrStride] per-XCD work counters, zero at launch
    const int32_t* pair_qid;    // the pairs grouped by cluster, each cluster's seeding (pass-1)
    const int32_t* pair_cid;    // pairs first: cluster c at [seg[c], seg[c + 1]), its seeding
                                // pairs at [seg[c], seg[nlist + 1 + c])
    const int32_t* seg;         // [2, nlist + 1] cluster starts, seeding ends
    int M;                      // pairs (both passes)
    int nlist;
    int unit_q;                 // queries per lower-bound unit (kUnitQ or kUnitQWide)
    const int2* groups;        // weight groups {first pair, pair count}
    const int32_t* grp_off;     // [nlist + 1]; grp_off[nlist] = number of groups
    int max_groups;
    int DP;                     // 64 * ceil(D_pad / 64): bytes per weight plane
    int8_t* pw;                 // [M, 2, DP] int8 weight planes (hi, lo), natural dim order
    PairRec* prec;              // [M]
    LbRec* lbr;                 // [M]
    int2* lbk;                  // [M] (kq, kq_pre) of lbr, packed for the scan's row loads
    const double* cbound;       // [nlist, kCbStride] (A_max, r_max, r_lo) per cluster
    const double* qep;          // [B] sum of qerr^2 per query
    double* tau;                // [B] float64 thresholds (set from the seeding lists)
    uint2* ub_list;             // [B, ub_cap] seeding bounds: each seeding unit's K smallest, as
                                // (bound bits with the row in the low 16, sorted position or -1)
    int32_t* ub_cnt;            // [B] entries appended to ub_list (may exceed ub_cap)
    uint32_t* ub_best;          // [B] smallest K-th bound of a unit whose entries did not fit
    int32_t* seed_cnt;          // [B] leading candidate slots already refined exactly (seeds)
    int ub_cap;
    float* tau_sq_out;          // [B] caller's float32 copy of the seeded tau, or null
    int xb_host;                // xb is mapped host memory (Stage Z reads cross PCIe)
    int use_l1;                 // residual-norm tile band: skip tiles no query can reach
    const float* tile_rmm;      // [tiles, 2] (min, max) of |x - c| per tile (use_l1)
    const float* pair_dqc;      // [M] |q - c| per pair (use_l1)
    int B;
    uint64_t* cand_key;
    int32_t* cand_id;
    int32_t* cand_cnt;
    int cap, K;
    unsigned long long* stats;  // [kStatSlots, 4] or null
    double rot_sq_min, rot_sq_max;
    double sum_rel;             // relative error bound of the per-pair float32 sums (sum_rel_of)
    // Fine level (used when the base is in host memory): per sorted row, 16-bit codes of x_rot
    // on the row's own grid and (offset, step, rho >= |x_rot - x_fine|), so that bounds within
    // ~1e-3 relative come from HBM instead of the exact row over PCIe.
    const uint16_t* fine_codes; // [N, D_pad] or null
    const float* fine_qp;       // [N, 4] (offset, step, rho, 0)
    int fine_mode;              // 1: seeds bounded and survivors filtered with the fine level
    int cm_emit;                // cm_scan_kernel: 1 lists rows, 0 only lowers the thresholds
    unsigned long long* host_rows;  // [1] rows read from the host-mapped base, or null
};

constexpr int kStatSlots = 64;  // telemetry counters are spread over this many [4] slots

__global__ void fill_i32_kernel(int32_t* p, int32_t v, int64_t n);
__global__ void copy_u64_kernel(const unsigned long long* src, unsigned long long* dst);

__global__ void stats_fold_kernel(const unsigned long long* slots, int64_t* out);

__global__ void prep_queries_kernel(const float* __restrict__ xq, int B, int D, int D_pad,
                                    const float* __restrict__ W, int ldw, int nlist,
                                    const float* __restrict__ bvec, double* __restrict__ xq64,
                                    double* __restrict__ xrot64, float* __restrict__ xrot32,
                                    double* __restrict__ qerr, int do_rot);

__global__ void coarse_dist_kernel(const double* __restrict__ xq64, int B, int D,
                                   const float* __restrict__ W, int ldw, int nlist,
                                   double* __restrict__ cd64);

__global__ void select_probes_kernel(const double* __restrict__ cd64, int nlist, int nprobe,
                                     int32_t* __restrict__ out_cids,
                                     float* __restrict__ out_dqcs, int ld,
                                     int32_t* __restrict__ out2_cids,
                                     float* __restrict__ out2_dqcs, int ld2);

template <int KP>
__global__ void select_probes_wave_kernel(const double* __restrict__ cd64, int B, int nlist,
                                          int nprobe, int32_t* __restrict__ out_cids,
                                          float* __restrict__ out_dqcs, int ld,
                                          int32_t* __restrict__ out2_cids,
                                          float* __restrict__ out2_dqcs, int ld2);

__global__ void count_pairs_kernel(const int32_t* __restrict__ probe_cids, int ld, int B,
                                   int nprobe, int p_init, int nlist, int32_t* counts);

__global__ void scan_pairs_kernel(const int32_t* counts, int nlist, int32_t* seg_off,
                                  int32_t* cursor);

// The cluster-major layout of the batched route, each cluster's pass-1 pairs followed by its
// pass-2 pairs: seg_off[c] = the cluster's first pair, seg_off[nlist + 1 + c] = its first pass-2
// pair (both rows end with M); cursor receives the two rows for the scatter.  Two launches of
// nblk = ceil(nlist / kBlock) <= kBlock blocks: in-block offsets and block totals, then carries.
__global__ void scan_pairs_joint_local_kernel(const int32_t* counts, int nlist, int32_t* seg_off,
                                              int32_t* blk_tot);
__global__ void scan_pairs_joint_carry_kernel(const int32_t* counts, int nlist,
                                              const int32_t* blk_tot, int nblk, int32_t* seg_off,
                                              int32_t* cursor);

__global__ void scatter_pairs_kernel(const int32_t* __restrict__ probe_cids,
                                     const float* __restrict__ probe_dqcs, int ld, int B,
                                     int nprobe, int p_init, int nlist, int32_t* cursor,
                                     int32_t* __restrict__ p1_cids, int32_t* __restrict__ p1_qids,
                                     float* __restrict__ p1_dqcs, int32_t* __restrict__ p2_cids,
                                     int32_t* __restrict__ p2_qids, float* __restrict__ p2_dqcs);

constexpr int kGroupChunk = 2048;  // (query, probe) entries per block of the LDS grouping
// band front end (frontend.hip)
__global__ void pad_queries_kernel(const float* __restrict__ xq, int B, int D, int Dq,
                                   float* __restrict__ qt32, float* __restrict__ qn32, int NS,
                                   uint16_t* __restrict__ qtb);
__global__ void centroid_bf16_kernel(const float* __restrict__ cm32, int nlist, int Dq, int NS,
                                     uint32_t* __restrict__ cmtb);
__global__ void pad_centroids_kernel(const float* __restrict__ W, int ldw, int nlist, int D,
                                     int Dq, float* __restrict__ cm32, float* __restrict__ cmt32,
                                     float* __restrict__ cn32,
                                     unsigned long long* __restrict__ cmax2);
__global__ void coarse_gemm_kernel(const float* __restrict__ qt32, const float* __restrict__ qn32,
                                   int B, const float* __restrict__ cmt32,
                                   const float* __restrict__ cn32, int nlist, int Dq,
                                   float* __restrict__ a32);
template <int KP, int V, bool STREAM>
__global__ void select_band_kernel(const float* __restrict__ a32, const double* __restrict__ xq64,
                                   const float* __restrict__ cm32,
                                   const unsigned long long* __restrict__ cmax_dev,
                                   double cmax_host, int B, int nlist, int D, int Dq,
                                   double kappa, double kabs, const float* __restrict__ tmin,
                                   int lda, int nprobe,
                                   int32_t* __restrict__ out_cids,
                                   float* __restrict__ out_dqcs, int ld,
                                   int32_t* __restrict__ out2_cids,
                                   float* __restrict__ out2_dqcs, int ld2);
constexpr int kGemmTiles = 4;  // coarse_gemm_kernel: 16-centroid tiles per wave
// coarse_gemm_bf16_kernel (Dq <= 128): 16-centroid tiles per stage; the run of stages per
// block is the longest that still gives a grid of about kStreamBlocks blocks
constexpr int kStageTiles = 2;
constexpr int kStreamBlocks = 5120;
// Dq <= 128 on the bfloat16 matrix cores (NS = ceil(Dq / 32) steps of the split operands)
template <int NS>
__global__ void coarse_gemm_bf16_kernel(const uint32_t* __restrict__ qtb,
                                        const float* __restrict__ qn32, int B,
                                        const uint32_t* __restrict__ cmtb,
                                        const float* __restrict__ cn32, int nlist, int run_stages,
                                        float* __restrict__ a32, float* __restrict__ tmin);
// relative and absolute dot-product bounds of the two coarse passes (select_band_kernel's E)
inline double band_kappa_f32(int Dq) { return (double)(Dq + 2) * 0x1p-23; }
inline int band_steps_bf16(int Dq) { return (Dq + 31) / 32; }
// row length (floats) of the bfloat16 coarse pass's approximations: nlist rounded up to 4, so
// that each tile's results are one aligned 16-byte store
__host__ __device__ inline int band_lda(int nlist) { return (nlist + 3) & ~3; }
inline double band_kappa_bf16(int Dq) {
    return (double)(32 * band_steps_bf16(Dq) + 4) * 0x1p-23 * (1.0 + 0x1p-5) + 3.125 * 0x1p-16;
}
inline double band_kabs_bf16(int Dq) { return (double)(32 * band_steps_bf16(Dq)) * 0x1p-100; }
// band front end: up to 32 x 64 approximations in registers (16 or 32 per lane); past that
// each wave filters its streamed row through an LDS list (faster from nlist 4096 on than 64
// values per lane in registers)
constexpr int kBandMaxNlist = 2048;
// from this many centroids on, the bfloat16 coarse pass also writes each query's 16-centroid
// tile minima and the streaming selector reads only the tiles that can hold band members
constexpr int kTileMinNlist = 8192;
inline int band_dq(int D) { return (D + 15) & ~15; }

constexpr int kCoarseQW = 4;       // queries per wave of coarse_dist_kernel
constexpr int kCoarseNC = 2;       // centroids per lane of coarse_dist_kernel
constexpr int kPrepQB = 4;         // queries per wave of prep_queries_kernel

// Dynamic LDS bytes of the LDS grouping kernels; they are used while this is <= 64 KiB.
inline size_t group_lds_bytes(int nlist) { return (size_t)2 * (nlist + 1) * sizeof(int32_t); }

__global__ void count_pairs_rank_kernel(const int32_t* __restrict__ probe_cids, int ld, int B,
                                        int nprobe, int p_init, int nlist, int32_t* counts,
                                        int32_t* __restrict__ rank);
__global__ void scatter_pairs_rank_kernel(const int32_t* __restrict__ probe_cids,
                                          const float* __restrict__ probe_dqcs, int ld, int B,
                                          int nprobe, int p_init, int nlist,
                                          const int32_t* __restrict__ seg_off,
                                          const int32_t* __restrict__ rank,
                                          int32_t* __restrict__ p1_cids, int32_t* __restrict__ p1_qids,
                                          float* __restrict__ p1_dqcs, int32_t* __restrict__ p2_cids,
                                          int32_t* __restrict__ p2_qids, float* __restrict__ p2_dqcs);

__global__ void count_pairs_lds_kernel(const int32_t* __restrict__ probe_cids, int ld, int B,
                                       int nprobe, int p_init, int nlist, int32_t* counts);

__global__ void scatter_pairs_lds_kernel(const int32_t* __restrict__ probe_cids,
                                         const float* __restrict__ probe_dqcs, int ld, int B,
                                         int nprobe, int p_init, int nlist, int32_t* cursor,
                                         int32_t* __restrict__ p1_cids,
                                         int32_t* __restrict__ p1_qids,
                                         float* __restrict__ p1_dqcs,
                                         int32_t* __restrict__ p2_cids,
                                         int32_t* __restrict__ p2_qids,
                                         float* __restrict__ p2_dqcs);

// Routes of pair_scan_kernel (one per reference mode family).
enum ScanKind {
    kScanCascade = 0,    // mode 2, Stage Y / Z
    kScanCascadeUb = 1,  // mode 2, Stage X seeding + Stage Y / Z
    kScanExact = 2,      // mode 10, every vector refined exactly
    kScanTribase = 3,    // mode 11, exact with the per-vector triangle-inequality skip
    kScanHat = 4         // modes 0 / 1, SQ8 reconstruction distance, no refinement
};

template <int KP, int KIND>
__global__ void pair_scan_kernel(ScanArgs a);

template <int KP>
__global__ void merge_kernel(MergeArgs a);

// Mode 0's rerank: one workgroup per query takes the M <= 256 entries of its merged list
// (kScanHat keys, sorted positions as ids), computes their canonical float64 distances and
// writes the K best by (distance, original id).
struct RerankArgs {
    int B, K, M;
    const uint64_t* list_key;  // [B, KP]
    const int32_t* list_id;
    int KP;
    const float* xb;
    const double* xq64;        // [B, D]
    int D;
    float* out_d;              // [B, K]
    int64_t* out_i;
    unsigned long long* host_rows;  // [1] rows read from a host-mapped base, or null
};

template <int KO>
__global__ void rerank_kernel(RerankArgs a);

// Batched-route work units: queries of one cluster x one slice of ~kSplitVec vectors (at most
// kMaxSplit slices per cluster).  Seeding units hold <= 16 of the cluster's pass-1 queries;
// lower-bound units hold <= kUnitQ (D_pad <= 256) or kUnitQWide of all its queries, both passes
// together, so a slice is read once per 128 (64) queries.  With q_c queries in cluster c,
// sum_c ceil(q_c / uq) <= M / uq + nlist, so a launch pair has at most kMaxSplit * (ceil(M_1 /
// 16) + ceil(M / 64) + 2 nlist) <= max_units_of(M) units for M = M_1 + M_2 pairs, whatever
// the split.
constexpr int kUnitQ = 128;
constexpr int kUnitQWide = 64;
constexpr int kUnitQ0 = 16;
// Slice length sv (vectors) of the units: the narrow layout's longer slices halve the units'
// fixed costs; the wide layout and mode 10's matrix-core scan keep shorter ones (their units do
// more work per vector, so shorter slices balance the workgroups better).
constexpr int kSplitVecNarrow = 2048;
constexpr int kSplitVec = 1024;
// Lower-bound units of the narrow layout over clusters of >= kLongSliceRows rows on average take
// slices twice as long: half the units' fixed costs (prologue, survivor flush) at configs[4]
// (6,100 rows per cluster: pass B -3 %); shorter searches keep the shorter slices, whose units
// balance the workgroups better near the end of the launch.
constexpr int kLongSliceRows = 4096;
constexpr int kMaxSplit = 8;
constexpr int kCtrStride = 32;  // int32 between per-XCD counters (one 128-byte line each)

// Weight groups: the 32 consecutive pairs of a cluster's segment that one lower-bound wave
// scans together share one weight scale (pairs 32 k .. 32 k + 31 of the segment; units start
// on such boundaries, seeding waves of 16 queries use half a group).
constexpr int kGroupQ = 32;
// Relative error bound of the batched route's per-pair float32 sums over D_pad terms (Q = sum
// (q - vmin)^2, sum |w|, |q|^2): n - 1 additions in any order, each rounding by <= 2^-24 of a
// partial sum of non-negative terms, give (n - 1) 2^-24 (1 + n 2^-24); the rounded difference
// q - vmin inside Q's terms adds 2^-23 (1 + 2^-24).  (D_pad + 4) 2^-24 covers both for
// D_pad <= 1024.
inline double sum_rel_of(int D_pad) { return (double)(D_pad + 4) * 0x1p-24; }
constexpr int kCbStride = 4;  // doubles per cluster in the per-cluster bound table
// Survivors a lower-bound wave queues in LDS before appending them to the candidate lists.
constexpr int kSurvQ = 512;

// Units of both passes for `pairs` (query, probe) pairs: bounded with the seeding pass's
// smaller units (16 queries) for every pair, since the split between the passes (p_init) is a
// search parameter that the workspace size does not know.
inline int64_t max_units_of(int64_t pairs, int64_t nlist) {
    return (int64_t)kMaxSplit *
           ((pairs + kUnitQ0 - 1) / kUnitQ0 + (pairs + kUnitQWide - 1) / kUnitQWide + 2 * nlist);
}

inline int64_t max_groups_of(int64_t pairs, int64_t nlist) {
    return (pairs + kGroupQ - 1) / kGroupQ + nlist;
}

// seed_all: the seeding units cover every pair of a cluster (TRIDENT_UB_SEED 2), not only its
// pass-1 pairs; seed_sl: the seeding units scan the first seed_sl slices of each cluster.
// Two launches of ceil(2 nlist / kBlock) blocks; blk_tot holds 2 * kBlock block totals.
// sv: the seeding units' slice length, svb: the lower-bound units'.
__global__ void unit_scan_local_kernel(const int32_t* seg, const int32_t* vec_off, int nlist,
                                       int uqB, int seed_all, int seed_sl, int sv, int svb,
                                       int32_t* unit_off, int32_t* grp_off, int32_t* blk_tot);
__global__ void unit_scan_carry_kernel(int nlist, const int32_t* blk_tot, int nblk,
                                       int32_t* unit_off, int32_t* grp_off);

__global__ void unit_fill_kernel(const int32_t* seg, const int32_t* vec_off, int nlist, int uqB,
                                 int seed_all, int sv, int svb, const int32_t* unit_off, int4* units, int max_units,
                                 const int32_t* grp_off, int2* groups, int max_groups);

__global__ void fill_u64_kernel(unsigned long long* p, unsigned long long v, int64_t n);

__global__ void tau_to_f32_kernel(const double* tau, float* out, int B);

template <int KS, int M>
__global__ void ub_scan_kernel(BatchArgs a);

// Survivors a wave of lb_scan_kernel queues in LDS before appending them.
constexpr int kLbQ = 64;

__global__ void lb_prep_kernel(BatchArgs a);

template <int KP, int DQ>
__global__ void ub_kth_kernel(BatchArgs a);

template <int DQ>
__global__ void fine_filter_kernel(BatchArgs a, int B);

template <int KP>
__global__ void fine_tau_kernel(BatchArgs a, int B);

// Parallel rescan of overflowed candidate lists (MergeArgs, ovf_par).
__global__ void ovf_collect_kernel(MergeArgs a);
template <int KP, bool UB>
__global__ void ovf_scan_kernel(MergeArgs a);
template <int KP>
__global__ void ovf_kth_kernel(MergeArgs a);

template <int KP>
__global__ void cm_seed_kernel(BatchArgs a, int B);

__global__ void fine_bounds_kernel(BatchArgs a, const int32_t* __restrict__ qids,
                                  const int64_t* __restrict__ spos, int n, double* lb, double* ub);

// Bounds a seeding unit lists per query: its K smallest, at most 64.
__host__ __device__ constexpr int ub_per_unit(int K) { return K < 64 ? K : 64; }

// Seeding-list slots per query: at most 3 seeding probes (trident_p_init_rule) x kMaxSplit
// slices, ub_per_unit(K) bounds each; a unit whose entries no longer fit offers its K-th bound
// to ub_best instead.
inline int64_t ub_cap_of(int64_t K) { return 3 * kMaxSplit * (int64_t)ub_per_unit((int)K); }

// Seeding bounds carry their row: the bound is rounded up to a multiple of 2^16 in its bit
// pattern (at most 2^-7 of its value) and the low 16 bits hold the row's index in the unit's
// slice, or kNoRow when the slice is longer or the bound is not finite.
constexpr uint32_t kNoRow = 0xffffu;

template <int KS>
__global__ void lb_scan_kernel(BatchArgs a);       // KS <= 4 (D_pad <= 256)

template <int KS>
__global__ void lb_scan_wide_kernel(BatchArgs a);  // 4 < KS <= 16

template <bool HOST, int DQ>
__global__ void refine_survivors_kernel(BatchArgs a, int B);

// Mode 10 on the float32 matrix cores (D_pad = 4 D4 <= 256, K <= 128): the lower-bound units of
// one launch (unit_beg / unit_end), each listing (lb, ub) keys of the rows that can still enter
// the top-K; a.ctr[0] is the work counter (zero at launch), a.ub_best the per-query thresholds
// (+inf at launch).
template <int D4>
__global__ void cm_scan_kernel(BatchArgs a);

// The same for 256 < D_pad <= 1024: dims in chunks of 128, query chunks reloaded per block.
__global__ void cm_scan_wide_kernel(BatchArgs a);

template <int KS>
__global__ void pair_prep_kernel(BatchArgs a);

// Waves [0, ncl) fill the per-cluster bounds, waves [ncl, ncl + B) the per-query state; block
// 0 clears unit_ctr when given.
__global__ void aux_bounds_kernel(BatchArgs a, int ncl, int B, double* cbound, double* qep,
                                  int32_t* unit_ctr);

__global__ void sq8_bounds_kernel(ScanArgs a, const int32_t* __restrict__ qids,
                                  const int32_t* __restrict__ cids,
                                  const int64_t* __restrict__ spos, int n, double* lb,
                                  double* ub);

// Dynamic LDS bytes of pair_scan_kernel for a given D / D_pad.
inline size_t scan_dyn_lds_bytes(int D, int D_pad) {
    return (size_t)D * sizeof(double) + (size_t)3 * D_pad * sizeof(float);
}

}  // namespace trident
