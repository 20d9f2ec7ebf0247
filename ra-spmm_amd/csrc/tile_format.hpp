// tile_format.hpp — host-side tile format shared by TC_DIRECT, COMMUNITY_TC
// and SEGMENT_HYBRID.
//
// Layout (all arrays flat, row-major):
//   win_rows[W*8]        output row of window slot (COMMUNITY_TC order; -1 pad)
//   block_offsets[W+1]   blocks of window w are [block_offsets[w], block_offsets[w+1])
//   atox[blocks*8]       B row (column of A) gathered by each 8x1 vector; -1 = padding
//   vals[blocks*64]      block values, [block][window slot r][vector k], fp16 or
//                        bf16 bits.  One 16-byte row per slot is exactly the
//                        8-element K-run an MFMA 16x16x32 lane consumes.
//   seg_window/seg_bbegin/seg_bend/seg_slot per segment (bit 31 of seg_window
//   marks a sole segment, seg_slot = -1) and split_windows/split_offsets for
//   the deterministic merge.  SEGMENT_HYBRID splits windows of more than 64
//   blocks (the reference rule); the other two kinds only windows of more
//   than kTileDirectSplitBlocks.
#pragma once

#include <cstdint>
#include <vector>

#include "../../include/ra_spmm.h"
#include "ra_internal.hpp"

struct ra_tile_host {
    int32_t kind = 0, M = 0, K = 0, N = 0, value_dtype = RA_DTYPE_F16;
    bool active = false;
    int64_t nnz = 0;          // stored entries after duplicate merge
    int64_t num_vectors = 0;  // distinct (window, column) pairs
    int32_t max_window_blocks = 0;
    int32_t value_scale_log2 = 0;  // fp16 values are stored as v * 2^s
    std::vector<int32_t> win_rows, block_offsets, atox;
    std::vector<uint16_t> vals;
    std::vector<int32_t> seg_window, seg_bbegin, seg_bend, seg_slot, split_windows, split_offsets;
    double build_ms = 0.0;
};

namespace ra {

constexpr int kTileWindow = 8;        // rows per window
constexpr int kTileVec = 8;           // vectors per block
constexpr int kTileSegBlocks = 64;    // SEGMENT_HYBRID: max blocks per segment
// TC_DIRECT / COMMUNITY_TC are scheduled the same way with a much larger
// limit: only extreme (hub) windows are split, so one wave never serialises
// thousands of blocks while the rest of the GPU idles.
constexpr int kTileDirectSplitBlocks = 512;
constexpr uint32_t kTileSoleFlag = 0x80000000u;

uint16_t f32_to_f16_rne(float f);
// Power-of-two scale 2^s for fp16 storage: maps max|v| near 2^14 so small
// values (e.g. 1/sqrt(d_i d_j) of hub pairs) stay out of the fp16 subnormal
// range while leaving 4x headroom below the fp16 maximum.
int32_t f16_value_scale_log2(float max_abs);
uint16_t f32_to_bf16_rne(float f);

ra_status tile_host_build(int32_t kind, const int32_t* rowptr, const int32_t* colind,
                          const float* vals, int32_t M, int32_t K, int32_t N, int32_t value_dtype,
                          ra_tile_host& out);

}  // namespace ra

// Device plan: the same arrays in HBM plus per-plan scratch.
struct ra_tile_plan {
    ra_tile_info info{};
    int32_t num_items = 0;  // segments (every kind is scheduled as segments)
    ra::DeviceBuffer block_offsets, atox, vals, win_rows, seg_window, seg_bbegin, seg_bend,
        seg_slot, split_windows, split_offsets;
    // Column partitions (info.col_parts > 1): items and split windows of
    // partition q are [part_items[q], part_items[q+1]) and
    // [part_splits[q], part_splits[q+1]); cells are q * num_windows + window.
    std::vector<int32_t> part_items{0, 0}, part_splits{0, 0};
    ra::DeviceBuffer bconv;    // B converted to fp16/bf16 (grown per K*ldb)
    ra::DeviceBuffer scratch;  // partial slots of split windows
    // FP32 route: the stored values as a CSR sorted by (row, column), derived
    // on the first FP32-route call (tile_f32_route.hip), and a
    // ZERO_OVERHEAD_CSR plan over it when the row lengths are skewed.
    bool f32_ready = false;
    int64_t f32_nnz = 0;
    int32_t f32_parts = 1;  // column ranges of the derived CSR (rowptr holds parts * M + 1)
    ra::DeviceBuffer f32_rowptr, f32_colind, f32_vals;
    ra_zo_plan* f32_zo = nullptr;
    ra_tile_plan() = default;
    ra_tile_plan(const ra_tile_plan&) = delete;
    ra_tile_plan& operator=(const ra_tile_plan&) = delete;
    ~ra_tile_plan() { ra_zo_plan_destroy(f32_zo); }
};

namespace ra {
// FP32 route of a tile plan: derive the CSR of the stored values once, then
// run CSR_DIRECT (or ZERO_OVERHEAD_CSR for skewed rows) on it.
ra_status tile_f32_prepare(ra_tile_plan* p, hipStream_t st);
ra_status tile_f32_run(ra_tile_plan* p, const float* B, float* C, int32_t N, hipStream_t st);
}  // namespace ra
