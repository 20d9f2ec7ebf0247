/*
 * ra_spmm.h — C ABI of the MI355X-native regime-aware SpMM engine.
 *
 * C = A * B with A an M x K CSR matrix (int32 rowptr/colind, fp32 values) and
 * B a dense K x N row-major matrix; C is dense M x N row-major fp32.
 *
 * Conventions
 *   - Pointers named d_* are device (HBM) pointers, h_* are host pointers.
 *   - Every kernel entry point is asynchronous on `stream` (a hipStream_t;
 *     NULL = the null stream) and writes EVERY element of C, so C may be
 *     uninitialised on entry.
 *   - Functions return ra_status; on failure ra_last_error() holds a
 *     thread-local, human-readable message.  No function throws.
 *   - Plan handles are opaque, owned by the caller, released with the
 *     matching *_destroy.  A plan keeps per-plan scratch, so one plan must not
 *     be run concurrently from two streams.
 *
 * Each declaration names the reference interface it replaces
 * (tariqaf/RA-SpMM, file:line).
 */
#ifndef RA_SPMM_H
#define RA_SPMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RA_SPMM_ABI_VERSION 1

/* Opaque stream handle: identical to hipStream_t (struct ihipStream_t*). */
typedef struct ihipStream_t* ra_stream_t;

typedef enum ra_status {
    RA_OK = 0,
    RA_ERR_INVALID_ARGUMENT = 1,
    RA_ERR_HIP = 2,           /* a HIP runtime call failed                 */
    RA_ERR_OUT_OF_MEMORY = 3,
    RA_ERR_UNSUPPORTED = 4,   /* shape/dtype combination not implemented   */
    RA_ERR_INACTIVE_PLAN = 5, /* tile plan built with N < 16               */
    RA_ERR_INTERNAL = 6
} ra_status;

typedef enum ra_dtype {
    RA_DTYPE_F32 = 0,
    RA_DTYPE_F16 = 1,
    RA_DTYPE_BF16 = 2
} ra_dtype;

/* Path ids keep the reference NextPath numbering (ra_common.h:76-95). */
typedef enum ra_path {
    RA_PATH_CSR_DIRECT = 0,
    RA_PATH_CSR_ADAPTIVE = 1,
    RA_PATH_STAGED_REUSE = 2,
    RA_PATH_TC_SPARSE = 3,
    RA_PATH_ROW_SPLIT_CUDA = 4,
    RA_PATH_TC_REORDERED = 5,
    RA_PATH_HYBRID_TC_CUDA = 6,
    RA_PATH_CUSPARSE = 7,          /* served by the baseline CSR kernel */
    RA_PATH_RODE_ENHANCED = 8,
    RA_PATH_VECTORIZED_COARSE = 9,
    RA_PATH_LOCALITY_TILED = 10,
    RA_PATH_TC_DIRECT = 11,
    RA_PATH_COMMUNITY_TC = 12,
    RA_PATH_ZERO_OVERHEAD_CSR = 13,
    RA_PATH_SEGMENT_HYBRID = 14,
    RA_PATH_COUNT = 15
} ra_path;

/* Rejection codes keep the reference RejectReason numbering (ra_common.h:145-159). */
typedef enum ra_reject {
    RA_REJECT_CHOSEN = 0,
    RA_REJECT_NOT_FEASIBLE = 1,
    RA_REJECT_LOW_FILL = 2,
    RA_REJECT_LOW_COVERAGE = 3,
    RA_REJECT_HIGH_SKEW = 4,
    RA_REJECT_SMALL_N = 5,
    RA_REJECT_INSUFFICIENT_NNZ = 6,
    RA_REJECT_LOW_OCCUPANCY = 7,
    RA_REJECT_LOW_DEGREE_SKEW = 8,
    RA_REJECT_NOT_STRONG_ENOUGH = 9,
    RA_REJECT_MARGIN_TOO_SMALL = 10,
    RA_REJECT_NOT_IN_PORTFOLIO = 11,
    RA_REJECT_UNKNOWN = 12
} ra_reject;

typedef enum ra_portfolio { RA_PORTFOLIO_MAIN = 0, RA_PORTFOLIO_FULL = 1 } ra_portfolio;

/* Threshold table of the seven-rule router. REFERENCE reproduces the
 * published decisions; MI355X is recalibrated from measurements on gfx950. */
typedef enum ra_router_table { RA_TABLE_REFERENCE = 0, RA_TABLE_MI355X = 1 } ra_router_table;

/* Tile-route precision: FP16 / BF16 MFMA, or the FP32-FMA route that replaces
 * the reference's TF32 path (gfx950 has no xf32 MFMA). */
typedef enum ra_tile_route {
    RA_TILE_ROUTE_F16 = 0,
    RA_TILE_ROUTE_BF16 = 1,
    RA_TILE_ROUTE_FP32 = 2
} ra_tile_route;

typedef enum ra_tile_kind {
    RA_TILE_TC_DIRECT = 0,
    RA_TILE_COMMUNITY_TC = 1,
    RA_TILE_SEGMENT_HYBRID = 2
} ra_tile_kind;

/* ------------------------------------------------------------------ misc */
int ra_abi_version(void);
const char* ra_status_string(ra_status status);
const char* ra_last_error(void);
/* Reference: next_path_name, ra_common.h:116-135. */
const char* ra_path_name(int32_t path);
/* Reference: reject_reason_str, ra_common.h:161-178. */
const char* ra_reject_name(int32_t code);

/* -------------------------------------------------------------- features
 * The four routing inputs from rowptr alone, in the reference's two forms.
 * ra_features_host is the two-pass form of the host path: sigma^2 =
 * sum (d - avg)^2 / M in ascending row order.  ra_features_device is the
 * moment form of the GPU path: var = max(0, S2/M - avg^2) from the exact
 * integers nnz and sum(deg^2) (ra_features_from_moments).  Both return zero
 * features when M <= 0 or K <= 0, as the reference does.  The two forms'
 * degree_cv differ by at most one float32 ulp, and only rarely (when the
 * exact CV lies within the moment form's cancellation error of a float32
 * rounding boundary).
 * Reference: compute_production_router_features, router/router_features.cpp:79-111
 *            compute_production_router_features_gpu, router/router_features_cuda.cu:51-92 */
typedef struct ra_features {
    int32_t M, K, N;
    int32_t max_deg;
    int64_t nnz;          /* rowptr[M] - rowptr[0]            */
    int64_t sum_deg_sq;   /* exact sum of squared row lengths */
    int64_t empty_rows;
    double avg;           /* nnz / M                          */
    double std_dev;       /* population std of row length     */
    float avg_nnz_per_row;
    float std_nnz_per_row;
    float degree_cv;
    float max_to_mean_ratio;
} ra_features;

ra_status ra_features_host(const int32_t* h_rowptr, int32_t M, int32_t K, int32_t N,
                           ra_features* out);
/* Returns once the result is on the host: the reduction's last kernel writes
 * it to mapped pinned memory, which the call polls, falling back to a
 * synchronisation of `stream` after ~200 us (work queued ahead, or an error).
 * Calls are serialised per process (per-device buffers); not capturable. */
ra_status ra_features_device(const int32_t* d_rowptr, int32_t M, int32_t K, int32_t N,
                             ra_stream_t stream, ra_features* out);
/* Diagnostic ("FULL") structural features of a CSR matrix: row-length skew,
 * 16x16 tile fill statistics, row-signature locality proxies and 16-row window
 * scores.  Host arrays; O(nnz log nnz); never used by the deployed decision.
 * Reference: compute_router_features, router/router_features.cpp:113-432;
 * analyze_matrix_fn, bindings/ra_bindings.cpp:1993-2049. */
typedef struct ra_diag_features {
    float avg_nnz_per_row, std_nnz_per_row, degree_cv, max_to_mean_ratio, frac_dense_rows,
        skew_ratio, long_row_fraction, long_row_nnz_fraction, top_1_row_nnz_fraction,
        top_5_row_nnz_fraction;
    float tile_fill_mean, tile_fill_median, tile_fill_p90, tile_fill_max, tile_fill_variance,
        tile_occupancy, actual_nnz_coverage, avg_nnz_per_tile, row_window_colspan_compactness,
        local_row_similarity_proxy, reordered_locality_proxy, locality_gain_proxy,
        locality_selectivity_proxy, road_likeness_proxy, row_split_affinity_proxy,
        mixedness_proxy;
    float tc_candidate_ratio, tc_synergy_proxy, estimated_tc_partition_ratio,
        estimated_cuda_partition_ratio, irregular_window_fraction, tc_granularity_proxy,
        redundancy_risk_proxy;
    int32_t tc_candidate_tiles;
    int32_t N, M, K;
    int64_t nnz;  /* rowptr[M] */
} ra_diag_features;

ra_status ra_analyze_matrix(const int32_t* h_rowptr, const int32_t* h_colind, int32_t M, int32_t K,
                            int32_t N, ra_diag_features* out);

/* Moment-form finalisation from exact integer moments (the device path's;
 * router/router_features_cuda.cu:83-91). */
ra_status ra_features_from_moments(int32_t M, int32_t K, int32_t N, int64_t nnz,
                                   int64_t sum_deg_sq, int32_t max_deg, int64_t empty_rows,
                                   ra_features* out);

/* ---------------------------------------------------------------- router
 * Reference: route_dispatch deployed block, router/router_dispatch.cpp:979-1110,
 *            feasibility router/router_dispatch.cpp:107-464. */
typedef struct ra_route {
    int32_t chosen_path;      /* ra_path                               */
    int32_t use_tf32;         /* run the tile path on its FP32 route   */
    int32_t rule;             /* 1..7 = matched rule, 8 = fallthrough  */
    int32_t tile_ok;
    float estimated_risk;
    float pad_;
    double est_plan_s;        /* preprocessing-aware tile-gate estimate */
    char decision_reason[64];
    int8_t feasible[RA_PATH_COUNT];
    int8_t rejection_code[RA_PATH_COUNT];
} ra_route;

ra_status ra_route_dispatch(const ra_features* features, int32_t portfolio, int32_t table,
                            ra_route* out);

/* ------------------------------------------------------------ CSR family */
/* CSR_DIRECT: lane-group-per-row SpMM for 64-lane wavefronts.
 * Reference: csr_direct_spmm, csr/csr_direct.cu:234-338 (binding spmm_csr_direct,
 *            bindings/ra_bindings.cpp:724-742). */
ra_status ra_spmm_csr_direct(const int32_t* d_rowptr, const int32_t* d_colind,
                             const float* d_vals, const float* d_B, float* d_C,
                             int32_t M, int32_t K, int32_t N, int64_t nnz,
                             ra_stream_t stream);

/* Hand-written regime-free baseline CSR kernel (one row per wavefront).
 * Replaces the cuSPARSE guardrail: CuSparseSpMMState, bindings/ra_bindings.cpp:431-615;
 * spmm_cusparse_fn, bindings/ra_bindings.cpp:821-836. */
ra_status ra_spmm_csr_baseline(const int32_t* d_rowptr, const int32_t* d_colind,
                               const float* d_vals, const float* d_B, float* d_C,
                               int32_t M, int32_t K, int32_t N, int64_t nnz,
                               ra_stream_t stream);
/* Precision-matched baseline: the same kernel with A values and B stored as
 * IEEE fp16 bits (d_vals_h [nnz], d_B_h [K,N]) and fp32 products and sums into
 * fp32 C.  Replaces the fp16 cuSPARSE guardrail (CuSparseSpMMState with
 * fp16 = true): spmm_cusparse_fp16_fn / benchmark_cusparse_fp16[_cold]_fn,
 * bindings/ra_bindings.cpp:895-960. */
ra_status ra_spmm_csr_baseline_f16(const int32_t* d_rowptr, const int32_t* d_colind,
                                   const uint16_t* d_vals_h, const uint16_t* d_B_h, float* d_C,
                                   int32_t M, int32_t K, int32_t N, int64_t nnz,
                                   ra_stream_t stream);

/* ZERO_OVERHEAD_CSR: O(M) degree binning, small-row lane groups, 256-nnz hub
 * chunks with a deterministic merge.
 * Reference: make_ra_zero_overhead_plan / run_ra_zero_overhead_plan,
 *            csr/ra_zero_overhead.cu:312-506; RAZeroOverheadPlan, ra_common.h:507-530. */
typedef struct ra_zo_plan ra_zo_plan;
typedef struct ra_zo_info {
    int32_t M, K;
    int32_t num_tiny, num_short, num_medium, num_long, num_empty;
    int32_t num_small;        /* tiny + short + medium                   */
    int32_t num_chunks;       /* 256-nnz chunks of rows with > 64 nnz    */
    int32_t num_sole_chunks;  /* rows of 65..256 nnz: one chunk, direct  */
    int32_t num_split_rows;   /* rows of > 256 nnz                       */
    int32_t num_split_chunks; /* their chunks (partial slots)            */
    int32_t max_long_chunks;
    int32_t pad_;
    int64_t plan_bytes;
} ra_zo_info;

/* Host-only binning (no device work): fills the lists the plan uploads.
 * small_rows: tiny, then short, then medium rows, each in ascending row order;
 * chunk_rows/chunk_starts: one entry per 256-nnz chunk, bit 31 of chunk_rows set
 * on sole chunks.  Any output pointer may be NULL; counts go to *info. */
ra_status ra_zo_bins_host(const int32_t* h_rowptr, int32_t M, int32_t K,
                          int32_t* small_rows, int32_t* chunk_rows, int32_t* chunk_starts,
                          int32_t* empty_rows, ra_zo_info* info);
ra_status ra_zo_plan_create(const int32_t* h_rowptr, int32_t M, int32_t K, ra_zo_plan** out);
/* Device binning of the same plan from a device rowptr (one scan on the GPU;
 * replaces the host O(M) loop of the reference's plan build).  Synchronises
 * `stream`.  Lists are identical to ra_zo_plan_create's. */
ra_status ra_zo_plan_create_device(const int32_t* d_rowptr, int32_t M, int32_t K, ra_stream_t stream,
                                   ra_zo_plan** out);
/* Copy a plan list to the host: "short_rows" (empty, tiny, short, medium rows),
 * "chunk_rows", "chunk_starts", "chunk_slot", "split_rows", "split_off".
 * dst may be NULL to query *count. */
ra_status ra_zo_plan_export(const ra_zo_plan* plan, const char* name, int32_t* dst, int64_t* count);
ra_status ra_zo_plan_run(ra_zo_plan* plan, const int32_t* d_rowptr, const int32_t* d_colind,
                         const float* d_vals, const float* d_B, float* d_C, int32_t N,
                         ra_stream_t stream);
/* Measurement hook (no reference counterpart): stage 1 runs only the fused
 * chunk + short-row kernel, stage 2 only the deterministic merge of split rows,
 * stage 0 both (== ra_zo_plan_run).  Lets a profiler time each launch alone. */
ra_status ra_zo_plan_run_stage(ra_zo_plan* plan, const int32_t* d_rowptr,
                               const int32_t* d_colind, const float* d_vals, const float* d_B,
                               float* d_C, int32_t N, int32_t stage, ra_stream_t stream);
/* No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same kernels and results as ra_zo_plan_run, but the partial
 * slots of rows longer than 256 nonzeros live in a fixed 64 MiB device array
 * of the library (one per GPU, held until the process ends) instead of a
 * plan-owned buffer, and no call allocates.  num_split_chunks * N * 4 bytes
 * must fit in 64 MiB, else RA_ERR_UNSUPPORTED.  Calls on one GPU share the
 * array: calls that overlap on one GPU race. */
ra_status ra_zo_plan_run_noalloc(ra_zo_plan* plan, const int32_t* d_rowptr,
                                 const int32_t* d_colind, const float* d_vals, const float* d_B,
                                 float* d_C, int32_t N, ra_stream_t stream);
ra_status ra_zo_plan_get_info(const ra_zo_plan* plan, ra_zo_info* info);
void ra_zo_plan_destroy(ra_zo_plan* plan);

/* ----------------------------------------------------------- tile family
 * 8-row windows; every distinct column of a window is an 8x1 vector; 8 vectors
 * form a block (the last one zero-padded).  COMMUNITY_TC first stable-sorts rows
 * by their leading column; SEGMENT_HYBRID splits windows with > 64 blocks into
 * <= 64-block segments merged deterministically.
 * Reference: build_ra_tc_direct_plan_impl, tc/ra_tc_direct.cu:627-780;
 *            make_ra_community_tc_plan, tc/ra_community_tc.cu:320-471;
 *            make_ra_segment_hybrid_plan, tc/ra_segment_hybrid.cu:371-543;
 *            run_* of the three files (tc/ra_tc_direct.cu:805-894,
 *            tc/ra_community_tc.cu:476-552, tc/ra_segment_hybrid.cu:548-668). */
typedef struct ra_tile_host ra_tile_host;
typedef struct ra_tile_plan ra_tile_plan;
typedef struct ra_tile_info {
    int32_t kind, M, K, active;
    int32_t num_windows;
    int32_t num_blocks;        /* reference num_tc_tiles                   */
    int32_t num_segments;
    int32_t num_split_windows;
    int32_t num_split_segs;
    int32_t max_window_blocks;
    int64_t nnz;
    int64_t num_vectors;       /* distinct (window, column) pairs          */
    int64_t plan_bytes;
    float avg_tile_density;    /* nnz / (values per block * num_blocks)    */
    int32_t value_dtype;       /* RA_DTYPE_F16 or RA_DTYPE_BF16            */
    double build_ms;           /* host build + upload                      */
    int32_t value_scale_log2;  /* fp16 plans store v * 2^s (s chosen from   */
                               /* max|v|), outputs are scaled back by 2^-s */
    int32_t rows_per_window;   /* 8: the reference's 8-row windows, blocks of
                                * 8 vectors; 16 or 32: tall windows, blocks of
                                * 32 vectors [rows/16][4][16][8] */
    int32_t col_parts;         /* 1, or P column ranges: windows are cut into
                                * P cells (partition-major) run one partition
                                * at a time, accumulating into C in order */
    int32_t pad3_;
} ra_tile_info;

/* Host-only build of the tile format (testable without a GPU).
 * value_dtype: RA_DTYPE_F16 or RA_DTYPE_BF16 (storage of the block values). */
ra_status ra_tile_host_build(int32_t kind, const int32_t* h_rowptr, const int32_t* h_colind,
                             const float* h_vals, int32_t M, int32_t K, int32_t N,
                             int32_t value_dtype, ra_tile_host** out);
ra_status ra_tile_host_get_info(const ra_tile_host* host, ra_tile_info* info);
/* Array export for structural checks. name: "block_offsets", "atox", "win_rows",
 * "vals" (uint16 bits, [block][row 8][vector 8]), "seg_window", "seg_bbegin",
 * "seg_bend", "seg_slot", "split_windows", "split_offsets".
 * Returns the element count in *count; copies when dst != NULL. */
ra_status ra_tile_host_export(const ra_tile_host* host, const char* name, void* dst,
                              int64_t* count);
void ra_tile_host_destroy(ra_tile_host* host);

ra_status ra_tile_plan_create(int32_t kind, const int32_t* h_rowptr, const int32_t* h_colind,
                              const float* h_vals, int32_t M, int32_t K, int32_t N,
                              int32_t value_dtype, ra_tile_plan** out);
/* Device build (sorts and scans on the GPU; the cold-path replacement of the
 * reference's host OpenMP build).  CSR arrays are device pointers; synchronises
 * `stream`.  rows_per_window: 8 gives the reference's format, bit-identical to
 * ra_tile_plan_create on the same input; 16 or 32 a tall format (more rows
 * share each gathered B row); 0 picks the height from the matrix (distinct
 * (row / h, column) counts and the kernel's memory-instruction cost). */
ra_status ra_tile_plan_create_device(int32_t kind, const int32_t* d_rowptr, const int32_t* d_colind,
                                     const float* d_vals, int32_t M, int32_t K, int32_t N,
                                     int32_t value_dtype, int32_t rows_per_window, ra_stream_t stream,
                                     ra_tile_plan** out);
/* Copy a plan array back to the host (same names as ra_tile_host_export). */
ra_status ra_tile_plan_export(const ra_tile_plan* plan, const char* name, void* dst,
                              int64_t* count);
/* B fp32 [K,N]; route: ra_tile_route.  The FP16/BF16 routes convert B into
 * plan scratch first (one extra pass over B).  RA_TILE_ROUTE_FP32 (the
 * reference's TF32 route, tc/ra_tc_direct.cu:805-894) computes exact fp32 fma
 * of the stored values as a CSR SpMM: its first call derives that CSR from the
 * plan on the device (allocates and synchronises `stream` once), later calls
 * only launch. */
ra_status ra_tile_plan_run(ra_tile_plan* plan, const float* d_B, float* d_C, int32_t N,
                           int32_t route, ra_stream_t stream);
/* B already fp16/bf16 with leading dimension ldb (elements, ldb >= N and a
 * multiple of 8): no conversion pass. */
ra_status ra_tile_plan_run_lowp(ra_tile_plan* plan, const void* d_Bh, int32_t ldb,
                                int32_t b_dtype, float* d_C, int32_t N, ra_stream_t stream);
ra_status ra_tile_plan_get_info(const ra_tile_plan* plan, ra_tile_info* info);
void ra_tile_plan_destroy(ra_tile_plan* plan);

/* ------------------------------------------------------------ utilities */
/* fp32 -> fp16/bf16 round-to-nearest-even conversion of a [rows, cols] matrix
 * into a buffer with leading dimension ldo (columns cols..ldo-1 zero-filled).
 * Reference: convert_b_to_half_kernel, tc/ra_tc_direct.cu:85-104. */
ra_status ra_convert_f32(const float* d_in, void* d_out, int64_t rows, int32_t cols,
                         int32_t ldo, int32_t out_dtype, ra_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RA_SPMM_H */
