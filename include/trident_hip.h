/*
 * trident_hip.h -- C ABI of libtrident_hip.so, the MI355X (gfx950) lossless IVF query path.
 *
 * Plain pointers and sizes only; no torch types.  Every device pointer may also be a
 * mapped pinned-host address (xb_sorted in the out-of-core mode).  Streams are passed as
 * `void*` holding a hipStream_t.  All entry points return TRIDENT_OK (0) or an error
 * code; trident_last_error() gives the message of the calling thread's last failure.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   trident_search          launch_trident_v4_search, src/trident_v4_kernels.cu:1172-1604
 *                           (modes 0, 1, 2, 10, 11), bound in Python at :1606-1627
 *   trident_coarse_probe    at::addmm_out coarse GEMM + trident_topk_centroids_kernel,
 *                           src/trident_v4_kernels.cu:1233-1259 and :68-162
 *   trident_group_pairs     trident_counting_sort_pairs_kernel, :168-263 (+ split :1264-1276)
 *   trident_sq8_bounds      the per-vector SQ8 lower/upper bound arithmetic of Stage Y / X,
 *                           :626-676 and :731-773 (exposed for bound-rigour tests)
 *   trident_host_alloc_mapped / trident_host_free / trident_host_device_pointer
 *                           the pinned host buffer of the out-of-core engine,
 *                           benchmarks/phase8_ooc_100m_4080.py:501-507 (torch pin_memory)
 */
#ifndef TRIDENT_HIP_H
#define TRIDENT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRIDENT_ABI_VERSION 6

enum TridentStatus {
    TRIDENT_OK = 0,
    TRIDENT_ERR_INVALID_ARGUMENT = 1,
    TRIDENT_ERR_UNSUPPORTED = 2,
    TRIDENT_ERR_WORKSPACE_TOO_SMALL = 3,
    TRIDENT_ERR_HIP = 4,
    TRIDENT_ERR_OUT_OF_MEMORY = 5
};

enum TridentMode {
    TRIDENT_MODE_SQ8_RERANK = 0, /* reference K0 / CM-SQ8+RR: top rerank_m by the SQ8 reconstruction
                                    distance, exact rerank to top-K (top-K by it when rerank_m = 0);
                                    approximate */
    TRIDENT_MODE_SQ8 = 1,        /* reference K1: top-K by the SQ8 reconstruction distance
                                    (acc_hat, returned as the distance); approximate */
    TRIDENT_MODE_CASCADE = 2,    /* Stage X (optional) + Stage Y SQ8 LB cascade + Stage Z exact refine */
    TRIDENT_MODE_CM_EXACT = 10,  /* cluster-major exhaustive exact scan (reference CM-FP32 route) */
    TRIDENT_MODE_TRIBASE = 11    /* exact scan skipping x with | |q-c| - |x-c| | > tau (reference
                                    Tribase-GPU); needs r_vec_sorted */
};

/* Device-resident index layout produced by trident_amd.TridentV4Index
 * (reference layout: benchmarks/phase4a_suite.py:95-278). */
typedef struct TridentIndexView {
    int32_t N, D, D_pad, nlist;
    int32_t tile_size;       /* vectors per tile, a multiple of 64 (64 or 256) */
    int32_t total_tiles;
    int32_t num_blocks;      /* SQ8 dimension blocks; blk_bounds4 holds num_blocks + 1 */
    int32_t per_cluster_sq8; /* 1: vmin/delta/eps_dim are [nlist, D_pad]; 0: [1, D_pad] */
    const float* W_combined; /* [D, ldw], ldw = nlist + D_pad: [-2 C^T | R | 0] */
    const float* b_combined; /* [ldw]: [|c|^2 | b | 0], rotation x -> x R + b */
    double rot_sq_min;       /* lower bound on the squared singular values of R */
    double rot_sq_max;       /* upper bound on the squared singular values of R */
    const uint32_t* sq8_packed;      /* [total_tiles, D_pad / 4, tile_size]; may be NULL when
                                        sq8_cells is set: mode 2 then takes the batched route
                                        only (the per-pair route, modes 0 / 1 and
                                        trident_sq8_bounds read it) */
    const int32_t* tile_orig_ids;    /* [total_tiles, tile_size], -1 padded */
    const float* tile_r_minmax;      /* [total_tiles, 2] residual-norm band, or NULL */
    const int32_t* cluster_tile_off; /* [nlist + 1] */
    const int32_t* cluster_vec_off;  /* [nlist + 1] */
    const float* xb_sorted;          /* [N, D] cluster-sorted base (device or mapped host) */
    const int32_t* orig_ids_sorted;  /* [N] */
    const float* vmin;               /* [nlist or 1, D_pad] */
    const float* delta;              /* [nlist or 1, D_pad] */
    const float* eps_dim;            /* [nlist or 1, D_pad] rigorous |x_rot - x_hat| bound */
    const int32_t* blk_bounds4;      /* [num_blocks + 1], device, in units of 4 dims */
    const float* vec_Ar;             /* [N, 2] sorted order: |code*delta|^2 rounded down (margin
                                        1e-13), residual-norm bound rounded up; NULL disables the
                                        batched route */
    const uint32_t* sq8_cells;       /* [total_tiles, tile_size / V, D_pad / 16, V, 4] with
                                        V = 64 for D_pad <= 256, else 16: the codes of
                                        sq8_packed regrouped as 16-byte cells (dims 16 g ..
                                        16 g + 15 of one slot), every byte c stored as c ^ 0x80
                                        (c - 128 as int8), each V-slot block contiguous; NULL
                                        disables the batched route */
    /* Centroids for the matrix-core coarse pass, Dq = D rounded up to 16, c_d = -W_combined[d, c]
     * / 2.  Optional (all or none): when cent_rows is NULL every search derives them from
     * W_combined into its workspace.  No counterpart in the reference (its coarse GEMM reads
     * W_coarse_only directly). */
    const float* cent_rows;          /* [nlist, Dq] zero-padded rows */
    const float* cent_tiles;         /* [ceil(nlist / 16) * 16 * Dq] matrix-core tile layout: float4
                                        (t Dq/16 + j) 64 + l holds dims (l / 16) Dq/4 + 4 j .. + 3
                                        of centroid 16 t + l % 16 */
    const float* cent_norms;         /* [nlist] float32(sum_d c_d^2) */
    double cent_norm_max;            /* max_c sum_d c_d^2 (float64) */
    const float* r_vec_sorted;       /* [N] |x - c(x)| in sorted order, float32 of the float64 norm
                                        (reference r_vec_sorted, src/trident_v4_kernels.cu:1216);
                                        mode 11 only, else may be NULL */
    /* Fine level (optional, both or none; no counterpart in the reference): 16-bit codes of
     * every rotated row on its own grid.  Used by the batched route when xb_sorted is mapped
     * host memory: the seeds' and the survivors' bounds then come from HBM within ~1e-3
     * relative, and only rows that can still enter the top-K cross PCIe. */
    const uint16_t* fine_codes;      /* [N, D_pad] sorted order: rint((x_rot - offset) / step) */
    const float* fine_qp;            /* [N, 4]: offset, step (x_fine = offset + code * step, one
                                        rounding in float64), rho >= |x_rot(exact) - x_fine|
                                        (rounded up), 0 */
    /* Per-cluster constants of the batched route's bounds (optional; no counterpart in the
     * reference): [nlist, 4] float64 filled once per index by trident_cluster_bounds.  When
     * NULL every batched search recomputes them, one pass over vec_Ar (8 N bytes). */
    const double* cluster_bounds;
    /* Per-row code norms of the batched route's lower-bound pass (optional; no counterpart in the
     * reference): [N] float32 in sorted order, >= sqrt(sum_d (code_d - 128)^2) over the D_pad
     * dims.  With them the pass bounds the lo weight plane's share of each row's sum by
     * Cauchy-Schwarz (the row's norm times the query block's largest lo-plane norm) instead of
     * 128 sum |lo|, so fewer tiles need the lo plane; NULL keeps the per-query bound. */
    const float* vec_cn;
    /* Rows of each seeding cluster the batched route's seeding pass scans (no counterpart in the
     * reference): 0 = one slice of up to 2048 rows (two slices past K = 64, or for a host base
     * without a fine level); a positive value caps each slice at max(512, seed_rows) rows (before
     * rounding up to 64), for an index whose rows within a cluster are ordered by residual norm,
     * so that a cluster's first rows are its best seeds.  Results do not depend on it. */
    int32_t seed_rows;
    /* The rows of xb_sorted as uint8 (optional; no counterpart in the reference): [N, D], for a
     * base whose every value is an integer in [0, 255] (the float32 values exactly), in the same
     * kind of memory as xb_sorted; needs D a multiple of 16 and a 16-byte aligned pointer.  The
     * batched route's and mode 10's exact refines (seeds and Stage Z) read these rows instead of
     * xb_sorted's: the same distances from a quarter of the bytes, which for a base in mapped
     * host memory are the bytes crossing PCIe.  NULL: every refine reads xb_sorted. */
    const uint8_t* xb_sorted_u8;
} TridentIndexView;

/* How modes 2 and 10 are executed.  Both routes are exact; they differ in speed only.  Mode 10
 * batched is the float32 matrix-core cluster-major scan: it needs K <= 128 and D_pad <= 1024
 * (AUTO takes it from 4 queries per probed cluster on average, and always for a base in mapped
 * host memory, where it reads each probed row once per unit instead of once per pair). */
enum TridentRoute {
    TRIDENT_ROUTE_AUTO = 0,     /* batched when clusters are shared by enough queries */
    TRIDENT_ROUTE_PAIR = 1,     /* one workgroup per (cluster, query): Stage X / Y / Z per pair
                                   (mode 10: the float64 scan of every row) */
    TRIDENT_ROUTE_BATCHED = 2   /* one workgroup per (cluster, query block): int8 matrix-core bound
                                   (mode 10: float32 matrix-core distances with an error band) */
};

typedef struct TridentSearchParams {
    int32_t mode;    /* TRIDENT_MODE_CASCADE or TRIDENT_MODE_CM_EXACT */
    int32_t B;       /* queries */
    int32_t K;       /* 1..128 */
    int32_t nprobe;  /* 1..min(nlist, 512) */
    int32_t ub_seed; /* TRIDENT_UB_SEED semantics: 0 off, 1 pass 1, 2 both passes */
    int32_t use_l1;  /* residual-norm tile band (needs tile_r_minmax) */
    int32_t p_init;  /* pass-1 probes per query; -1 = reference rule */
    int32_t route;   /* TridentRoute (modes 2 and 10) */
    int32_t rerank_m; /* mode 0: candidates reranked exactly, M = min(max(rerank_m, K), 200);
                         0 = no rerank.  Ignored by the other modes */
} TridentSearchParams;

/* Stage boundaries at which trident_search records the caller's events (if given). */
enum TridentStageEvent {
    TRIDENT_EV_START = 0,       /* before the front end */
    TRIDENT_EV_PROBED = 1,      /* rotation + coarse distances + top-nprobe done */
    TRIDENT_EV_GROUPED = 2,     /* pairs grouped by cluster */
    TRIDENT_EV_P1_SCAN = 3,     /* pass-1 pair scan done */
    TRIDENT_EV_P1_MERGE = 4,    /* pass-1 merge (threshold) done */
    TRIDENT_EV_P2_SCAN = 5,     /* pass-2 pair scan done */
    TRIDENT_EV_END = 6,         /* final merge done */
    TRIDENT_EV_COUNT = 7
};

typedef struct TridentSearchOutputs {
    float* topk_d;        /* [B, K] squared L2 distances (float32), +inf if missing */
    int64_t* topk_i;      /* [B, K] original ids, -1 if missing */
    int32_t* probe_cids;  /* [B, probe_ld] probed clusters in (d, cid) order, or NULL */
    float* probe_dqcs;    /* [B, probe_ld] |q - c| of each probe, or NULL */
    int32_t probe_ld;     /* row stride of probe_cids / probe_dqcs (>= nprobe) */
    int32_t n_events;     /* entries in `events` (<= TRIDENT_EV_COUNT) */
    float* tau_sq;        /* [B] pass-1 threshold (squared, rounded up), or NULL */
    int64_t* stats;       /* [4] candidates, scanned dims, survivors, refined-inserted; or NULL */
    void* const* events;  /* hipEvent_t handles recorded at TridentStageEvent points, or NULL */
    int64_t* host_rows;   /* [1] base rows read from a host-mapped xb_sorted (4*D bytes each, over
                             PCIe: exact seeds, Stage Z, overflow rescans), or NULL */
    int64_t* host_rows_seed; /* [1] the part of host_rows read by the first (seeding) pass:
                                the exact seeds of the batched route, the first pass of the
                                per-pair route; 0 for a device base; or NULL.  No reference
                                counterpart (its per-pass PCIe split came from a profiler). */
} TridentSearchOutputs;

/* Timing events for TridentSearchOutputs.events (hipEventCreate / Destroy / ElapsedTime). */
int trident_event_create(void** event);
int trident_event_destroy(void* event);
int trident_event_elapsed_ms(void* start, void* stop, float* ms);

/* Bytes of scratch trident_search needs for batches up to max_B x max_nprobe x max_K.  For mode 0
 * with rerank_m > 0, max_K must cover M = min(max(rerank_m, K), 200) as well. */
size_t trident_workspace_bytes(const TridentIndexView* ix, int32_t max_B, int32_t max_nprobe,
                               int32_t max_K);

/* Full batched query: front end, two-pass scan, merge.  Asynchronous on `stream`. */
int trident_search(const TridentIndexView* ix, const TridentSearchParams* sp, const float* xq,
                   void* workspace, size_t workspace_bytes, const TridentSearchOutputs* out,
                   void* stream);

/* Bytes of the fixed scratch array behind trident_search_noalloc (one per GPU, 64 MiB). */
#define TRIDENT_NOALLOC_SCRATCH_BYTES (64u << 20)

/* trident_search without a workspace argument, and without any allocation: its scratch memory
 * is a fixed device array of TRIDENT_NOALLOC_SCRATCH_BYTES compiled into the library (one copy
 * per GPU, kept until the process ends).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under graph capture, tight serving loops, hosts that
 * forbid hipMalloc).  Batches whose trident_workspace_bytes exceeds the array fail with
 * TRIDENT_ERR_WORKSPACE_TOO_SMALL.  The stream's device must be the current device.  Every call
 * on one GPU shares that GPU's array (each call initialises what it reads), so calls that
 * overlap on one GPU -- on different streams or host threads -- race and must be serialised by
 * the caller; calls in one stream are ordered and safe. */
int trident_search_noalloc(const TridentIndexView* ix, const TridentSearchParams* sp,
                           const float* xq, const TridentSearchOutputs* out, void* stream);

/* Front end only: float64 coarse distances and the exact (d, cid) top-nprobe per query.
 * workspace: >= trident_workspace_bytes(ix, B, nprobe, 1) bytes. */
int trident_coarse_probe(const TridentIndexView* ix, const float* xq, int32_t B, int32_t nprobe,
                         void* workspace, size_t workspace_bytes, int32_t* probe_cids,
                         float* probe_dqcs, int32_t probe_ld, void* stream);

/* Group (cluster, query) pairs by cluster for the two passes.  probe_cids: [B, probe_ld].
 * Outputs pass p (0, 1): pair_cids[p] / pair_qids[p] of length B * (p ? nprobe - p_init :
 * p_init), and seg_off[p][nlist + 1] cluster segment offsets.  counts_ws: 2 * (nlist + 1)
 * int32 scratch. */
int trident_group_pairs(const int32_t* probe_cids, int32_t probe_ld, int32_t B, int32_t nprobe,
                        int32_t p_init, int32_t nlist, int32_t* p1_cids, int32_t* p1_qids,
                        int32_t* p2_cids, int32_t* p2_qids, int32_t* seg_off,
                        int32_t* counts_ws, void* stream);

/* The reference two-pass split rule (src/trident_v4_kernels.cu:1264-1276): mode 0 by rerank_m,
 * modes 1 / 2 / 11 by B, K and nprobe, mode 10 single-pass. */
int32_t trident_p_init_rule(int32_t mode, int32_t B, int32_t K, int32_t nprobe, int32_t rerank_m);

/* The route (TRIDENT_ROUTE_PAIR or TRIDENT_ROUTE_BATCHED) a mode-2 trident_search with these
 * sizes and requested route takes, or a negative error code when the request cannot run.
 * No reference counterpart: the reference has a single per-pair kernel; this lets a caller
 * (or a benchmark) know which kernels its search launches. */
int32_t trident_route_for(const TridentIndexView* ix, int32_t B, int32_t K, int32_t nprobe,
                          int32_t requested_route);

/* As trident_route_for for mode 2 or mode 10 (for mode 10 TRIDENT_ROUTE_BATCHED is the float32
 * matrix-core scan, which also depends on where xb_sorted lives); other modes take the per-pair
 * route.  No reference counterpart. */
int32_t trident_route_for_mode(const TridentIndexView* ix, int32_t mode, int32_t B, int32_t K,
                               int32_t nprobe, int32_t requested_route);

/* Per-candidate SQ8 bounds exactly as Stage Y (lb) and Stage X (ub) evaluate them, scaled to
 * bound the canonical float64 distance: lb[i] <= d64(q, x) <= ub[i] for the n (query,
 * sorted-position) pairs.  cids/qids/spos are device arrays of length n. */
int trident_sq8_bounds(const TridentIndexView* ix, const float* xq, int32_t B,
                       const int32_t* qids, const int32_t* cids, const int64_t* spos, int32_t n,
                       void* workspace, size_t workspace_bytes, double* lb, double* ub,
                       void* stream);

/* Fills cluster_bounds ([nlist, 4] float64, device) from delta, eps_dim and vec_Ar: per cluster
 * A_max >= every |code * delta|^2, r_max >= every stored residual bound, r_lo = the smallest
 * stored residual bound.  No reference counterpart (index-constant part of the batched route's
 * bounds, hoisted out of the search). */
int trident_cluster_bounds(const TridentIndexView* ix, double* cluster_bounds, void* stream);

/* The fine-level bounds the out-of-core search uses, for (query, sorted-position) pairs:
 * lb[i] <= d64(q, x) <= ub[i].  No reference counterpart (exposed for bound-rigour tests).
 * workspace: >= trident_workspace_bytes(ix, B, 1, 1) bytes. */
int trident_fine_bounds(const TridentIndexView* ix, const float* xq, int32_t B,
                       const int32_t* qids, const int64_t* spos, int32_t n, void* workspace,
                       size_t workspace_bytes, double* lb, double* ub, void* stream);

/* Pinned, device-mapped host memory for the out-of-core base. */
int trident_host_alloc_mapped(size_t bytes, void** host_ptr);
int trident_host_free(void* host_ptr);
int trident_host_device_pointer(void* host_ptr, void** device_ptr);

const char* trident_last_error(void);
int trident_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TRIDENT_HIP_H */
