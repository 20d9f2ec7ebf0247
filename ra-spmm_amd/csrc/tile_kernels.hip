// tile_kernels.hip — TC_DIRECT / COMMUNITY_TC / SEGMENT_HYBRID on gfx950.
//
// Work item = one window (TC_DIRECT, COMMUNITY_TC) or one segment
// (SEGMENT_HYBRID): 8 output rows and a run of blocks [b0, b1).
//
// FP16/BF16 route (tile_mfma_kernel): one wavefront per (item, 16*CPL-column
// slice), v_mfma_f32_16x16x32_{f16,bf16}.  A step consumes 4 blocks (32
// vectors = the MFMA K).  Lane (j = lane & 15, q = lane >> 4):
//   - gathers B rows atox[(b+q)*8 + v], v < 8, CPL contiguous elements each at
//     columns col0 + j*CPL (one 16-byte load per vector for CPL = 8), then
//     transposes in registers so MFMA number cc sees K = vectors, N = column
//     col0 + j*CPL + cc;
//   - feeds block b+q as the A fragment in block-diagonal form: rows 0-7 of the
//     16-row MFMA carry blocks b, b+1 and rows 8-15 carry b+2, b+3, so an 8-row
//     window fills the 16x16x32 shape; the two halves are summed at the end.
// FP32 route (the `_tf32` entry points): replaces the reference's TF32 path
// (gfx950 has no xf32 MFMA) with exact fp32 FMA of the stored fp16/bf16 values
// and fp32 B, run as a CSR SpMM over the plan's stored values
// (tile_f32_route.hip).
//
// Reference: fs_tile_spmm[_staged]_kernel tc/ra_tc_direct.cu:109-179, 270-328;
//            ct_fs_tile_spmm_perm_kernel tc/ra_community_tc.cu:106-190;
//            sh_fs_tile_spmm_seg_kernel / sh_merge_split_kernel
//            tc/ra_segment_hybrid.cu:90-221; convert_b_to_half_kernel
//            tc/ra_tc_direct.cu:85-104.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>

#include "ra_internal.hpp"
#include "tile_format.hpp"

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int CPL> struct HalfRun;  // CPL contiguous 16-bit elements
template <> struct HalfRun<1> { typedef unsigned short T; };
template <> struct HalfRun<2> { typedef unsigned short T __attribute__((ext_vector_type(2))); };
template <> struct HalfRun<4> { typedef unsigned short T __attribute__((ext_vector_type(4))); };
template <> struct HalfRun<8> { typedef u16x8 T; };

template <int CPL>
__device__ __forceinline__ unsigned short run_elem(const typename HalfRun<CPL>::T& r, int i) {
    if constexpr (CPL == 1) return r;
    else return r[i];
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma32(u16x8 a, u16x8 b, f32x4 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

struct Items {
    const int32_t* block_offsets;
    const int32_t* seg_window;
    const int32_t* seg_bbegin;
    const int32_t* seg_bend;
    const int32_t* seg_slot;
    const int32_t* win_rows;       // COMMUNITY_TC
    int item_base;                 // first segment of this launch
    int cell_base;                 // partition * windows (column partitions)
    int accumulate;                // add into C (partitions after the first)
};

// Write (or, for later column partitions, add) one output value / 16-byte run.
__device__ __forceinline__ void put1(float* dst, float v, bool add) {
    if (add) v += *dst;
    *dst = v;
}
template <typename V4>
__device__ __forceinline__ void put4(float* dst, V4 v, bool add) {
    if (add) v += *reinterpret_cast<const V4*>(dst);
    __builtin_nontemporal_store(v, reinterpret_cast<V4*>(dst));
}

// Work item i = segment i (a whole window unless the window was split).
__device__ __forceinline__ void item_range(const Items& it, int i, int& w, int& b0, int& b1,
                                           int& slot) {
    i += it.item_base;
    w = static_cast<int>(static_cast<uint32_t>(it.seg_window[i]) & 0x7FFFFFFFu) - it.cell_base;
    b0 = it.seg_bbegin[i];
    b1 = it.seg_bend[i];
    slot = it.seg_slot[i];
}

// Destination of window slot m (0..H-1): a C row, or a partial-slot row.
template <int KIND, int H = ra::kTileWindow>
__device__ __forceinline__ float* item_row(const Items& it, float* C, float* scratch, int w,
                                           int slot, int m, int M, int N) {
    if (slot >= 0) return scratch + ((int64_t)slot * H + m) * N;
    int row;
    if constexpr (KIND == RA_TILE_COMMUNITY_TC) row = it.win_rows[(int64_t)w * H + m];
    else row = w * H + m;
    if (row < 0 || row >= M) return nullptr;
    return C + (int64_t)row * N;
}

// 1-D grid: block -> (group of 4 items, column slice), slice fastest, so all
// slices of a window run back to back and share its atox/vals in L2.  With
// remap on, each XCD (workgroups are dealt round-robin over 8) takes one
// contiguous range of windows, keeping neighbouring windows in one L2.
// order bit 0: XCD remap; bit 1: slice slowest (all windows of slice 0, then
// slice 1, ...), which shrinks the gathered working set to one slice of each
// B row when B is far larger than the L2.
__device__ __forceinline__ void tile_block_coords(int nslices, int order, int64_t& item_blk,
                                                  int& slice) {
    int64_t bid = blockIdx.x;
    if (order & 1) {
        const int64_t nb = gridDim.x, q = nb / 8, r = nb % 8, x = bid % 8, k = bid / 8;
        bid = x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
    }
    if (order & 2) {
        const int64_t per_slice = gridDim.x / nslices;
        slice = static_cast<int>(bid / per_slice);
        item_blk = bid - (int64_t)slice * per_slice;
    } else {
        item_blk = bid / nslices;
        slice = static_cast<int>(bid - item_blk * nslices);
    }
}

// ------------------------------------------------------------ MFMA route
template <int CPL, bool BF16, int KIND>
__global__ __launch_bounds__(kBlock) void tile_mfma_kernel(
    Items it, const int32_t* __restrict__ atox, const uint16_t* __restrict__ vals,
    const uint16_t* __restrict__ Bh, int ldb, float* __restrict__ C, float* __restrict__ scratch,
    int M, int N, int num_items, int nslices, int remap, float unscale, int vec_store) {
    typedef typename HalfRun<CPL>::T Run;
    const int lane = threadIdx.x & (kWave - 1);
    int64_t item_blk;
    int slice;
    tile_block_coords(nslices, remap, item_blk, slice);
    const int item = __builtin_amdgcn_readfirstlane(
        static_cast<int>(item_blk * kWavesPerBlock + (threadIdx.x >> 6)));
    if (item >= num_items) return;
    int w, b0, b1, slot;
    item_range(it, item, w, b0, b1, slot);
    const int j = lane & 15;
    const int q = lane >> 4;
    const int col = slice * (16 * CPL) + j * CPL;
    const bool col_ok = col < ldb;  // ldb % 8 == 0 and CPL | 8: whole run in bounds
    const bool a_half = (j < 8) == (q < 2);

    f32x4 acc[CPL];
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) acc[cc] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Column indices come 32 blocks (8 steps) at a time: one 16-byte load per
    // lane (lane L: indices 4L..4L+3, half L&1 of block c0 + L/2), handed to
    // step s's lane group q (block c0 + 4s + q) from lanes 8s + 2q and
    // 8s + 2q + 1 by lane permutes, which use the LDS unit, not the address
    // unit.  A fragments come two steps per load: lane j needs block b+q's
    // row j&7 on even steps when a_half, and its partner lane j^8 (same q and
    // row, !a_half) loads the same row of block b+4+q, handed over on the odd
    // step by a lane exchange.  The pair is loaded one step ahead.
    auto load_chunk = [&](int c0) {
        int4 v = make_int4(-1, -1, -1, -1);
        if (c0 + (lane >> 1) < b1) v = *reinterpret_cast<const int4*>(atox + (int64_t)c0 * 8 + lane * 4);
        return v;
    };
    auto load_pair = [&](int b) {  // b = first block of an even step
        const int blk = b + q + (a_half ? 0 : 4);
        u16x8 a = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        if (blk < b1) a = *reinterpret_cast<const u16x8*>(vals + (int64_t)blk * 64 + (j & 7) * 8);
        return a;
    };
    int4 chunk = load_chunk(b0), chunk_next = make_int4(-1, -1, -1, -1);
    u16x8 apair = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (b0 < b1) apair = load_pair(b0);
    for (int b = b0; b < b1; b += 4) {
        const int t = (b - b0) >> 2;
        const int s = t & 7;
        if (s == 0 && b + 32 < b1) chunk_next = load_chunk(b + 32);  // one chunk ahead
        const int l0 = 8 * s + 2 * q;
        int cols[8];
        cols[0] = __shfl(chunk.x, l0, kWave);
        cols[1] = __shfl(chunk.y, l0, kWave);
        cols[2] = __shfl(chunk.z, l0, kWave);
        cols[3] = __shfl(chunk.w, l0, kWave);
        cols[4] = __shfl(chunk.x, l0 + 1, kWave);
        cols[5] = __shfl(chunk.y, l0 + 1, kWave);
        cols[6] = __shfl(chunk.z, l0 + 1, kWave);
        cols[7] = __shfl(chunk.w, l0 + 1, kWave);
        u16x8 a;
        if ((t & 1) == 0) {
            a = a_half ? apair : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        } else {
            // The partner's register holds this step's row of block b+q.
            const u32x4 mine = __builtin_bit_cast(u32x4, apair);
            u32x4 o;
            o[0] = __shfl_xor(mine[0], 8, kWave);
            o[1] = __shfl_xor(mine[1], 8, kWave);
            o[2] = __shfl_xor(mine[2], 8, kWave);
            o[3] = __shfl_xor(mine[3], 8, kWave);
            a = a_half ? __builtin_bit_cast(u16x8, o) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        Run raw[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            if (cols[v] >= 0 && col_ok)
                raw[v] = *reinterpret_cast<const Run*>(Bh + (int64_t)cols[v] * ldb + col);
            else
                raw[v] = Run{};
        }
        if ((t & 1) == 1 && b + 4 < b1) apair = load_pair(b + 4);
        if (s == 7) chunk = chunk_next;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) {
            u16x8 bop;
#pragma unroll
            for (int v = 0; v < 8; ++v) bop[v] = run_elem<CPL>(raw[v], cc);
            acc[cc] = mfma32<BF16>(a, bop, acc[cc]);
        }
    }

    // D[m][n]: lane holds rows 4*(lane>>4)+r, column n = lane & 15.  Rows m and
    // m+8 are partial sums of the same window row (block-diagonal A): lanes L
    // and L^32 exchange them, so both halves hold the window's sums and each
    // half stores two of its four rows (every lane stores).
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[cc][r] += __shfl_xor(acc[cc][r], 32, kWave);
    // The lane's CPL columns are contiguous: 16-byte streaming stores when the
    // rows allow it (C is written once and never read back here).
    const bool vec = (CPL % 4 == 0) && vec_store && col + CPL <= N;
    const bool upper = lane >= 32;  // rows 2, 3 of the lane's group of four
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int m = 4 * ((lane >> 4) & 1) + (upper ? 2 : 0) + k;
        float out[CPL];
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) out[cc] = (upper ? acc[cc][2 + k] : acc[cc][k]) * unscale;  // exact
        float* dst = item_row<KIND>(it, C, scratch, w, slot, m, M, N);
        if (!dst) continue;
        const bool add = it.accumulate && slot < 0;
        if constexpr (CPL % 4 == 0) {
            if (vec) {
#pragma unroll
                for (int cc = 0; cc < CPL; cc += 4)
                    put4(dst + col + cc, f32x4{out[cc], out[cc + 1], out[cc + 2], out[cc + 3]}, add);
                continue;
            }
        }
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc)
            if (col + cc < N) put1(dst + col + cc, out[cc], add);
    }
}


// ------------------------------------------------- MFMA route, tall windows
// Windows of H = 16*RG rows; a block is 32 vectors (one MFMA K) with values
// [RG][4][16][8]: lane (j, q) of row group g loads the 16-byte run of row
// 16g + j over vectors 8q..8q+7.  Every gathered B row feeds RG MFMAs (one per
// row group), so a B row shared by several of the H rows is gathered once.
// Per step: one index load (lane pairs exchange halves), 8 B-row gathers,
// RG A loads; no block-diagonal padding.
template <int CPL, bool BF16, int KIND, int RG>
__global__ __launch_bounds__(kBlock) void tile_mfma_tall_kernel(
    Items it, const int32_t* __restrict__ atox, const uint16_t* __restrict__ vals,
    const uint16_t* __restrict__ Bh, int ldb, float* __restrict__ C, float* __restrict__ scratch,
    int M, int N, int num_items, int nslices, int order, float unscale, int vec_store) {
    typedef typename HalfRun<CPL>::T Run;
    constexpr int H = 16 * RG;
    constexpr int BV = H * 32;  // values per block
    const int lane = threadIdx.x & (kWave - 1);
    int64_t item_blk;
    int slice;
    tile_block_coords(nslices, order, item_blk, slice);
    const int item = __builtin_amdgcn_readfirstlane(
        static_cast<int>(item_blk * kWavesPerBlock + (threadIdx.x >> 6)));
    if (item >= num_items) return;
    int w, b0, b1, slot;
    item_range(it, item, w, b0, b1, slot);
    const int j = lane & 15;
    const int q = lane >> 4;
    const int col = slice * (16 * CPL) + j * CPL;
    const bool col_ok = col < ldb;

    f32x4 acc[RG][CPL];
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) acc[g][cc] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Column indices come 8 blocks at a time: one 16-byte load per lane
    // covers the 256 indices of blocks [c0, c0 + 8) (lane L: indices 4L..4L+3),
    // and step b takes its 8 from lanes 8s + 2q and 8s + 2q + 1 (s = b - c0)
    // by lane permutes, which use the LDS unit, not the address unit.
    auto load_chunk = [&](int c0) {
        int4 v = make_int4(-1, -1, -1, -1);
        if (c0 + (lane >> 3) < b1) v = *reinterpret_cast<const int4*>(atox + (int64_t)c0 * 32 + lane * 4);
        return v;
    };
    auto cols_of = [&](const int4& chunk, int s, int (&cols)[8]) {
        const int l0 = 8 * s + 2 * q;
        cols[0] = __shfl(chunk.x, l0, kWave);
        cols[1] = __shfl(chunk.y, l0, kWave);
        cols[2] = __shfl(chunk.z, l0, kWave);
        cols[3] = __shfl(chunk.w, l0, kWave);
        cols[4] = __shfl(chunk.x, l0 + 1, kWave);
        cols[5] = __shfl(chunk.y, l0 + 1, kWave);
        cols[6] = __shfl(chunk.z, l0 + 1, kWave);
        cols[7] = __shfl(chunk.w, l0 + 1, kWave);
    };
    auto load_a = [&](int b, u16x8 (&a)[RG]) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
            a[g] = *reinterpret_cast<const u16x8*>(vals + (int64_t)b * BV + ((g * 4 + q) * 16 + j) * 8);
    };
    int4 chunk = load_chunk(b0), chunk_next = make_int4(-1, -1, -1, -1);
    u16x8 a_next[RG];
    if (b0 < b1) load_a(b0, a_next);
    for (int b = b0; b < b1; ++b) {
        const int s = (b - b0) & 7;
        if (s == 0 && b + 8 < b1) chunk_next = load_chunk(b + 8);  // one chunk ahead
        int cols[8];
        cols_of(chunk, s, cols);
        u16x8 a[RG];
#pragma unroll
        for (int g = 0; g < RG; ++g) a[g] = a_next[g];
        Run raw[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            if (cols[v] >= 0 && col_ok)
                raw[v] = *reinterpret_cast<const Run*>(Bh + (int64_t)cols[v] * ldb + col);
            else
                raw[v] = Run{};
        }
        if (b + 1 < b1) load_a(b + 1, a_next);
        if (s == 7) chunk = chunk_next;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) {
            u16x8 bop;
#pragma unroll
            for (int v = 0; v < 8; ++v) bop[v] = run_elem<CPL>(raw[v], cc);
#pragma unroll
            for (int g = 0; g < RG; ++g) acc[g][cc] = mfma32<BF16>(a[g], bop, acc[g][cc]);
        }
    }

    // D of row group g: lane holds rows 16g + 4q + r, column j's CPL outputs.
    const bool vec = (CPL % 4 == 0) && vec_store && col + CPL <= N;
#pragma unroll
    for (int g = 0; g < RG; ++g) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 16 * g + 4 * q + r;
            float* dst = item_row<KIND, H>(it, C, scratch, w, slot, m, M, N);
            if (!dst) continue;
            float out[CPL];
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc) out[cc] = acc[g][cc][r] * unscale;  // exact: power of two
            const bool add = it.accumulate && slot < 0;
            if constexpr (CPL % 4 == 0) {
                if (vec) {
#pragma unroll
                    for (int cc = 0; cc < CPL; cc += 4)
                        put4(dst + col + cc, f32x4{out[cc], out[cc + 1], out[cc + 2], out[cc + 3]}, add);
                    continue;
                }
            }
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc)
                if (col + cc < N) put1(dst + col + cc, out[cc], add);
        }
    }
}

// ------------------------------ MFMA route, 32-row windows on 32x32x16 MFMA
// The 32-row tall layout run with v_mfma_f32_32x32x16_{f16,bf16}: lane
// (j = lane & 31, q = lane >> 5) feeds row j over k = 8q..8q+7 of a half block
// (16 vectors) as the A operand and gathers B columns col0 + 8j .. +7 of those
// 8 vectors (one 16-byte load each, register transpose) as the B operand.  A
// wave covers 256 columns: each 64-lane gather reads 2 B rows of 512 bytes
// instead of 4 rows of 256 bytes, and a block's A values are read once per
// 256 columns instead of once per 128.  D of MFMA cc: lane holds rows
// 8(i/4) + 4q + i%4 (i < 16) of column col0 + 8j + cc.
template <bool BF16>
__device__ __forceinline__ f32x16 mfma3232(u16x8 a, u16x8 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF16, int KIND>
__global__ __launch_bounds__(kBlock, 2) void tile_mfma_tall32_kernel(
    Items it, const int32_t* __restrict__ atox, const uint16_t* __restrict__ vals,
    const uint16_t* __restrict__ Bh, int ldb, float* __restrict__ C, float* __restrict__ scratch,
    int M, int N, int num_items, int nslices, int order, float unscale, int vec_store) {
    constexpr int H = 32;
    constexpr int BV = H * 32;  // values per block
    const int lane = threadIdx.x & (kWave - 1);
    int64_t item_blk;
    int slice;
    tile_block_coords(nslices, order, item_blk, slice);
    const int item = __builtin_amdgcn_readfirstlane(
        static_cast<int>(item_blk * kWavesPerBlock + (threadIdx.x >> 6)));
    if (item >= num_items) return;
    int w, b0, b1, slot;
    item_range(it, item, w, b0, b1, slot);
    const int j = lane & 31;
    const int q = lane >> 5;
    const int col = slice * 256 + j * 8;
    const bool col_ok = col < ldb;
    // A operand of row j, k-group q4: offset in the [2][4][16][8] block layout.
    const int a_row = ((j >> 4) * 4) * 16 + (j & 15);

    f32x16 acc[8];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[cc][i] = 0.f;

    // Column indices: one 16-byte load per lane covers blocks [c0, c0 + 8);
    // block s, k-group q4 sits in lanes 8s + 2q4 and 8s + 2q4 + 1.
    auto load_chunk = [&](int c0) {
        int4 v = make_int4(-1, -1, -1, -1);
        if (c0 + (lane >> 3) < b1) v = *reinterpret_cast<const int4*>(atox + (int64_t)c0 * 32 + lane * 4);
        return v;
    };
    int4 chunk = load_chunk(b0), chunk_next = make_int4(-1, -1, -1, -1);
    for (int b = b0; b < b1; ++b) {
        const int s = (b - b0) & 7;
        if (s == 0 && b + 8 < b1) chunk_next = load_chunk(b + 8);
#pragma unroll 1
        for (int h = 0; h < 2; ++h) {
            const int q4 = 2 * h + q;
            int cols[8];
            const int l0 = 8 * s + 2 * q4;
            cols[0] = __shfl(chunk.x, l0, kWave);
            cols[1] = __shfl(chunk.y, l0, kWave);
            cols[2] = __shfl(chunk.z, l0, kWave);
            cols[3] = __shfl(chunk.w, l0, kWave);
            cols[4] = __shfl(chunk.x, l0 + 1, kWave);
            cols[5] = __shfl(chunk.y, l0 + 1, kWave);
            cols[6] = __shfl(chunk.z, l0 + 1, kWave);
            cols[7] = __shfl(chunk.w, l0 + 1, kWave);
            const u16x8 a = *reinterpret_cast<const u16x8*>(vals + (int64_t)b * BV + (a_row + q4 * 16) * 8);
            u16x8 raw[8];
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                if (cols[v] >= 0 && col_ok)
                    raw[v] = *reinterpret_cast<const u16x8*>(Bh + (int64_t)cols[v] * ldb + col);
                else
                    raw[v] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
#pragma unroll
            for (int cc = 0; cc < 8; ++cc) {
                u16x8 bop;
#pragma unroll
                for (int v = 0; v < 8; ++v) bop[v] = raw[v][cc];
                acc[cc] = mfma3232<BF16>(a, bop, acc[cc]);
            }
        }
        if (s == 7) chunk = chunk_next;
    }

    const bool vec = vec_store && col + 8 <= N;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i >> 2) + 4 * q + (i & 3);
        float* dst = item_row<KIND, H>(it, C, scratch, w, slot, m, M, N);
        if (!dst) continue;
        float out[8];
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) out[cc] = acc[cc][i] * unscale;  // exact: power of two
        const bool add = it.accumulate && slot < 0;
        if (vec) {
            put4(dst + col, f32x4{out[0], out[1], out[2], out[3]}, add);
            put4(dst + col + 4, f32x4{out[4], out[5], out[6], out[7]}, add);
        } else {
#pragma unroll
            for (int cc = 0; cc < 8; ++cc)
                if (col + cc < N) put1(dst + col + cc, out[cc], add);
        }
    }
}

// ------------------------------------------------ SEGMENT_HYBRID merge
// C[w*8+m][n] = ((slot0 + slot1) + ...) in ascending slot order
// (tc/ra_segment_hybrid.cu:198-221).
__global__ __launch_bounds__(kBlock) void tile_merge_kernel(
    const int32_t* __restrict__ split_windows, const int32_t* __restrict__ split_offsets,
    const int32_t* __restrict__ win_rows, const float* __restrict__ scratch, float* __restrict__ C,
    int M, int N, int H, int cell_base, int accumulate) {
    const int sw = blockIdx.x;
    const int o0 = split_offsets[sw], o1 = split_offsets[sw + 1];
    // grid.y is capped by the launch; stride over the window's H*N elements.
    for (int64_t e = (int64_t)blockIdx.y * kBlock + threadIdx.x; e < (int64_t)H * N;
         e += (int64_t)gridDim.y * kBlock) {
        const int m = static_cast<int>(e / N);
        const int n = static_cast<int>(e - (int64_t)m * N);
        const int64_t slot_row = (int64_t)(split_windows[sw] - cell_base) * H + m;
        const int row = win_rows ? win_rows[slot_row] : static_cast<int>(slot_row);
        if (row < 0 || row >= M) continue;
        float acc = scratch[((int64_t)o0 * H + m) * N + n];
        for (int o = o0 + 1; o < o1; ++o) acc += scratch[((int64_t)o * H + m) * N + n];
        if (accumulate) acc = C[(int64_t)row * N + n] + acc;
        C[(int64_t)row * N + n] = acc;
    }
}

// --------------------------------------------------------------- convert
// fp32 [rows, cols] -> 16-bit [rows, ldo], RNE, columns cols..ldo-1 zeroed.
// One thread writes 8 consecutive outputs (one 16-byte store); VEC reads them
// as two 16-byte loads (cols % 8 == 0, 16-byte aligned input).
template <bool BF16, bool VEC>
__global__ __launch_bounds__(kBlock) void convert_kernel(const float* __restrict__ in,
                                                         uint16_t* __restrict__ out, int64_t rows,
                                                         int cols, int ldo) {
    const int groups = ldo / 8;
    const int64_t total = rows * groups;
    for (int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x; g < total;
         g += (int64_t)gridDim.x * kBlock) {
        const int64_t r = g / groups;
        const int c0 = static_cast<int>(g - r * groups) * 8;
        const float* src = in + r * cols;
        float x[8];
        if constexpr (VEC) {
            const f32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + c0));
            const f32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + c0 + 4));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = lo[i];
                x[4 + i] = hi[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = (c0 + i < cols) ? src[c0 + i] : 0.f;
        }
        u16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (BF16) o[i] = __builtin_bit_cast(unsigned short, static_cast<__bf16>(x[i]));
            else o[i] = __builtin_bit_cast(unsigned short, static_cast<_Float16>(x[i]));
        }
        *reinterpret_cast<u16x8*>(out + r * ldo + c0) = o;
    }
}

ra_status launch_convert(const float* in, void* out, int64_t rows, int32_t cols, int32_t ldo,
                         bool bf16, hipStream_t st) {
    if (rows <= 0 || ldo <= 0) return RA_OK;
    const int64_t total = rows * (ldo / 8);
    const int blocks = static_cast<int>(std::min<int64_t>((total + kBlock - 1) / kBlock, 1 << 16));
    const bool vec = (cols % 8 == 0) && ldo == cols && ra::aligned16(in);
    uint16_t* o = static_cast<uint16_t*>(out);
    if (bf16 && vec) convert_kernel<true, true><<<blocks, kBlock, 0, st>>>(in, o, rows, cols, ldo);
    else if (bf16) convert_kernel<true, false><<<blocks, kBlock, 0, st>>>(in, o, rows, cols, ldo);
    else if (vec) convert_kernel<false, true><<<blocks, kBlock, 0, st>>>(in, o, rows, cols, ldo);
    else convert_kernel<false, false><<<blocks, kBlock, 0, st>>>(in, o, rows, cols, ldo);
    RA_LAUNCH_CHECK("convert_kernel");
    return RA_OK;
}

}  // namespace

namespace {

// RA_TILE_XCD_REMAP=0 turns the XCD-contiguous window order off.  It is never
// used for COMMUNITY_TC: the leading-column order clusters the heavy rows at
// the front, and contiguous ranges would hand all of them to one XCD.
int tile_remap() {
    static const int r = [] {
        const char* e = std::getenv("RA_TILE_XCD_REMAP");
        return e ? (std::atoi(e) != 0) : 1;
    }();
    return r;
}

// RA_TILE_CPL caps the columns per lane of the MFMA kernel (1, 2, 4 or 8):
// fewer columns per lane = fewer registers = more resident waves.
int tile_max_cpl() {
    static const int c = [] {
        const char* e = std::getenv("RA_TILE_CPL");
        const int v = e ? std::atoi(e) : 8;
        return v >= 8 ? 8 : v >= 4 ? 4 : v >= 2 ? 2 : 1;
    }();
    return c;
}

// RA_TILE_SLICE_MAJOR: 1 = always, 0 = never; unset = with the XCD window
// remap on and the row split into 4 or more slices (N > 384), where the
// whole-row working set is 4x the slice's.  Measured on C4 N=512 with 8 column
// partitions: TC_DIRECT (remapped) 14.4 -> 9.5 ms with slice-major order;
// COMMUNITY_TC (never remapped) 9.85 -> 8.94 ms without it.  At 2 slices the
// re-read A stream cancels the gain.
int tile_slice_major(int nslices, bool remapped) {
    static const int r = [] {
        const char* e = std::getenv("RA_TILE_SLICE_MAJOR");
        return e ? (std::atoi(e) != 0 ? 1 : 0) : -1;
    }();
    return r >= 0 ? r : (nslices >= 4 && remapped ? 1 : 0);
}

// One launch's share of a plan: all of it, or one column partition.
struct Part {
    int item_base, num_items, cell_base, accumulate, split_base, num_splits;
};

Part whole_plan(const ra_tile_plan* p) {
    return Part{0, p->num_items, 0, 0, 0, p->info.num_split_windows};
}

Items plan_items(const ra_tile_plan* p, const Part& part) {
    Items it{};
    it.item_base = part.item_base;
    it.cell_base = part.cell_base;
    it.accumulate = part.accumulate;
    it.block_offsets = p->block_offsets.get<int32_t>();
    it.seg_window = p->seg_window.get<int32_t>();
    it.seg_bbegin = p->seg_bbegin.get<int32_t>();
    it.seg_bend = p->seg_bend.get<int32_t>();
    it.seg_slot = p->seg_slot.get<int32_t>();
    it.win_rows = p->win_rows.get<int32_t>();
    return it;
}

template <int KIND>
ra_status launch_mfma_kind(const ra_tile_plan* p, const Part& part, const uint16_t* Bh, int ldb, bool bf16,
                           float* C, float* scratch, int N, hipStream_t st) {
    const int M = p->info.M;
    const Items it = plan_items(p, part);
    int cpl = N <= 16 ? 1 : N <= 32 ? 2 : N <= 64 ? 4 : 8;
    cpl = std::min(cpl, tile_max_cpl());
    const int nslices = (N + 16 * cpl - 1) / (16 * cpl);
    const int remap = (KIND == RA_TILE_COMMUNITY_TC ? 0 : tile_remap()) | (tile_slice_major(nslices, KIND != RA_TILE_COMMUNITY_TC && tile_remap()) ? 2 : 0);
    const float unscale = std::ldexp(1.0f, -p->info.value_scale_log2);
    dim3 grid(static_cast<unsigned>(((int64_t)part.num_items + kWavesPerBlock - 1) / kWavesPerBlock * nslices));
    const int vec_store = (N % 4 == 0) && ra::aligned16(C) && (!scratch || ra::aligned16(scratch));
#define RA_MFMA_CASE(c)                                                                            \
    if (cpl == c) {                                                                                \
        if (bf16)                                                                                  \
            tile_mfma_kernel<c, true, KIND><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(),    \
                p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, remap, unscale, vec_store); \
        else                                                                                       \
            tile_mfma_kernel<c, false, KIND><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(),   \
                p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, remap, unscale, vec_store); \
    }
    RA_MFMA_CASE(1)
    RA_MFMA_CASE(2)
    RA_MFMA_CASE(4)
    RA_MFMA_CASE(8)
#undef RA_MFMA_CASE
    RA_LAUNCH_CHECK("tile_mfma_kernel");
    return RA_OK;
}

ra_status launch_merge(const ra_tile_plan* p, const Part& part, float* C, int N, hipStream_t st) {
    if (part.num_splits == 0) return RA_OK;
    const int H = p->info.rows_per_window;
    dim3 grid(part.num_splits,
              static_cast<unsigned>(std::min<int64_t>(((int64_t)H * N + kBlock - 1) / kBlock, 65535)));
    const int32_t* wr = p->info.kind == RA_TILE_COMMUNITY_TC ? p->win_rows.get<int32_t>() : nullptr;
    tile_merge_kernel<<<grid, kBlock, 0, st>>>(p->split_windows.get<int32_t>() + part.split_base,
                                               p->split_offsets.get<int32_t>() + part.split_base, wr,
                                               p->scratch.get<float>(), C, p->info.M, N, H, part.cell_base,
                                               part.accumulate);
    RA_LAUNCH_CHECK("tile_merge_kernel");
    return RA_OK;
}

template <int KIND, int RG>
ra_status launch_mfma_tall(const ra_tile_plan* p, const Part& part, const uint16_t* Bh, int ldb, bool bf16,
                           float* C, float* scratch, int N, hipStream_t st) {
    const int M = p->info.M;
    const Items it = plan_items(p, part);
    int cpl = N <= 16 ? 1 : N <= 32 ? 2 : N <= 64 ? 4 : 8;
    cpl = std::min(cpl, tile_max_cpl());
    const int nslices = (N + 16 * cpl - 1) / (16 * cpl);
    const int order = (KIND == RA_TILE_COMMUNITY_TC ? 0 : tile_remap()) | (tile_slice_major(nslices, KIND != RA_TILE_COMMUNITY_TC && tile_remap()) ? 2 : 0);
    const float unscale = std::ldexp(1.0f, -p->info.value_scale_log2);
    dim3 grid(static_cast<unsigned>(((int64_t)part.num_items + kWavesPerBlock - 1) / kWavesPerBlock * nslices));
    const int vec_store = (N % 4 == 0) && ra::aligned16(C) && (!scratch || ra::aligned16(scratch));
#define RA_TALL_CASE(c)                                                                                  \
    if (cpl == c) {                                                                                      \
        if (bf16)                                                                                        \
            tile_mfma_tall_kernel<c, true, KIND, RG><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(), \
                p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, order, unscale, vec_store); \
        else                                                                                             \
            tile_mfma_tall_kernel<c, false, KIND, RG><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(), \
                p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, order, unscale, vec_store); \
    }
    RA_TALL_CASE(1)
    RA_TALL_CASE(2)
    RA_TALL_CASE(4)
    RA_TALL_CASE(8)
#undef RA_TALL_CASE
    RA_LAUNCH_CHECK("tile_mfma_tall_kernel");
    return RA_OK;
}

// 32-row windows run on the 32x32x16 MFMA kernel at N >= 512 (C3 N=512:
// 1.048 -> 0.968 ms; at N=256 its two waves per SIMD, one per window, lose:
// 0.498 -> 0.533 ms).  RA_TILE_MFMA32=1 forces it at N > 128, 0 turns it off.
bool tile_use_mfma32(int N) {
    static const int v = [] {
        const char* e = std::getenv("RA_TILE_MFMA32");
        return e ? std::atoi(e) : -1;
    }();
    if (v == 0) return false;
    if (v == 1) return N > 128;
    return N >= 512;
}

template <int KIND>
ra_status launch_mfma_tall32(const ra_tile_plan* p, const Part& part, const uint16_t* Bh, int ldb, bool bf16,
                             float* C, float* scratch, int N, hipStream_t st) {
    const int M = p->info.M;
    const Items it = plan_items(p, part);
    const int nslices = (N + 255) / 256;
    const int order = (KIND == RA_TILE_COMMUNITY_TC ? 0 : tile_remap()) |
                      (tile_slice_major(nslices, KIND != RA_TILE_COMMUNITY_TC && tile_remap()) ? 2 : 0);
    const float unscale = std::ldexp(1.0f, -p->info.value_scale_log2);
    dim3 grid(static_cast<unsigned>(((int64_t)part.num_items + kWavesPerBlock - 1) / kWavesPerBlock * nslices));
    const int vec_store = (N % 4 == 0) && ra::aligned16(C) && (!scratch || ra::aligned16(scratch));
    if (bf16)
        tile_mfma_tall32_kernel<true, KIND><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(),
            p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, order, unscale, vec_store);
    else
        tile_mfma_tall32_kernel<false, KIND><<<grid, kBlock, 0, st>>>(it, p->atox.get<int32_t>(),
            p->vals.get<uint16_t>(), Bh, ldb, C, scratch, M, N, part.num_items, nslices, order, unscale, vec_store);
    RA_LAUNCH_CHECK("tile_mfma_tall32_kernel");
    return RA_OK;
}

template <int KIND>
ra_status launch_kind(const ra_tile_plan* p, const Part& part, const uint16_t* Bh, int ldb, bool bf16, float* C,
                      float* scratch, int N, hipStream_t st) {
    if (part.num_items == 0) return RA_OK;
    switch (p->info.rows_per_window) {
        case 16:
            return launch_mfma_tall<KIND, 1>(p, part, Bh, ldb, bf16, C, scratch, N, st);
        case 32:
            if (tile_use_mfma32(N)) return launch_mfma_tall32<KIND>(p, part, Bh, ldb, bf16, C, scratch, N, st);
            return launch_mfma_tall<KIND, 2>(p, part, Bh, ldb, bf16, C, scratch, N, st);
        default:
            return launch_mfma_kind<KIND>(p, part, Bh, ldb, bf16, C, scratch, N, st);
    }
}

// FP16/BF16 MFMA route over 16-bit B (converted, or passed in by the caller).
ra_status run_common(ra_tile_plan* p, const uint16_t* Bh, int ldb, bool bf16, float* C, int N, hipStream_t st) {
    float* scratch = nullptr;
    if (p->info.num_split_segs > 0) {
        RA_TRY(p->scratch.ensure((size_t)p->info.num_split_segs * p->info.rows_per_window * N * sizeof(float)));
        scratch = p->scratch.get<float>();
    }
    // Column partitions run one after another on the stream, each adding into
    // C what the earlier ones wrote: the per-element sum order is fixed.
    const int P = std::max(p->info.col_parts, 1);
    for (int q = 0; q < P; ++q) {
        const Part part = P == 1 ? whole_plan(p)
                                 : Part{p->part_items[q], p->part_items[q + 1] - p->part_items[q],
                                        q * p->info.num_windows, q > 0 ? 1 : 0, p->part_splits[q],
                                        p->part_splits[q + 1] - p->part_splits[q]};
        switch (p->info.kind) {
            case RA_TILE_TC_DIRECT:
                RA_TRY(launch_kind<RA_TILE_TC_DIRECT>(p, part, Bh, ldb, bf16, C, scratch, N, st));
                break;
            case RA_TILE_COMMUNITY_TC:
                RA_TRY(launch_kind<RA_TILE_COMMUNITY_TC>(p, part, Bh, ldb, bf16, C, scratch, N, st));
                break;
            default:
                RA_TRY(launch_kind<RA_TILE_SEGMENT_HYBRID>(p, part, Bh, ldb, bf16, C, scratch, N, st));
                break;
        }
        RA_TRY(launch_merge(p, part, C, N, st));
    }
    return RA_OK;
}

}  // namespace

extern "C" {

ra_status ra_convert_f32(const float* d_in, void* d_out, int64_t rows, int32_t cols, int32_t ldo,
                         int32_t out_dtype, ra_stream_t stream) {
    if (rows < 0 || cols < 0 || ldo < cols || (ldo % 8) != 0)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "convert: need ldo >= cols and ldo % 8 == 0");
    if (out_dtype != RA_DTYPE_F16 && out_dtype != RA_DTYPE_BF16)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "convert: out_dtype must be F16 or BF16");
    if (rows > 0 && (!d_in || !d_out)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "convert: NULL buffer");
    if (!ra::aligned16(d_out)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "convert: output not 16-byte aligned");
    return launch_convert(d_in, d_out, rows, cols, ldo, out_dtype == RA_DTYPE_BF16,
                          reinterpret_cast<hipStream_t>(stream));
}

ra_status ra_tile_plan_create(int32_t kind, const int32_t* h_rowptr, const int32_t* h_colind,
                              const float* h_vals, int32_t M, int32_t K, int32_t N,
                              int32_t value_dtype, ra_tile_plan** out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: out is NULL");
    *out = nullptr;
    const auto t0 = std::chrono::steady_clock::now();
    ra_tile_host host;
    try {
        RA_TRY(ra::tile_host_build(kind, h_rowptr, h_colind, h_vals, M, K, N, value_dtype, host));
    } catch (const std::bad_alloc&) {
        return ra::fail(RA_ERR_OUT_OF_MEMORY, "tile: host build out of memory");
    }
    auto p = new (std::nothrow) ra_tile_plan();
    if (!p) return ra::fail(RA_ERR_OUT_OF_MEMORY, "tile: plan allocation");
    ra_status s = ra_tile_host_get_info(&host, &p->info);
    if (s == RA_OK && host.active) {
        if ((s = p->block_offsets.upload(host.block_offsets)) == RA_OK &&
            (s = p->atox.upload(host.atox)) == RA_OK && (s = p->vals.upload(host.vals)) == RA_OK &&
            (s = p->win_rows.upload(host.win_rows)) == RA_OK &&
            (s = p->seg_window.upload(host.seg_window)) == RA_OK &&
            (s = p->seg_bbegin.upload(host.seg_bbegin)) == RA_OK &&
            (s = p->seg_bend.upload(host.seg_bend)) == RA_OK &&
            (s = p->seg_slot.upload(host.seg_slot)) == RA_OK &&
            (s = p->split_windows.upload(host.split_windows)) == RA_OK &&
            (s = p->split_offsets.upload(host.split_offsets)) == RA_OK) {
            p->num_items = p->info.num_segments;
        }
    }
    if (s != RA_OK) {
        delete p;
        return s;
    }
    p->info.build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    *out = p;
    return RA_OK;
}

ra_status ra_tile_plan_run(ra_tile_plan* p, const float* d_B, float* d_C, int32_t N, int32_t route,
                           ra_stream_t stream) {
    if (!p) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: plan is NULL");
    if (!p->info.active)
        return ra::fail(RA_ERR_INACTIVE_PLAN, "tile: plan is inactive (built with N < 16 or empty matrix)");
    if (N <= 0 || p->info.M == 0) return RA_OK;
    if (!d_B || !d_C) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: NULL B or C");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (route == RA_TILE_ROUTE_FP32) return ra::tile_f32_run(p, d_B, d_C, N, st);
    if (route != RA_TILE_ROUTE_F16 && route != RA_TILE_ROUTE_BF16)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: unknown route");
    const bool bf16 = route == RA_TILE_ROUTE_BF16;
    if (bf16 != (p->info.value_dtype == RA_DTYPE_BF16))
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: route precision differs from the plan's value dtype");
    const int ldb = (N + 7) / 8 * 8;
    RA_TRY(p->bconv.ensure((size_t)p->info.K * ldb * sizeof(uint16_t)));
    RA_TRY(launch_convert(d_B, p->bconv.get(), p->info.K, N, ldb, bf16, st));
    return run_common(p, p->bconv.get<uint16_t>(), ldb, bf16, d_C, N, st);
}

ra_status ra_tile_plan_run_lowp(ra_tile_plan* p, const void* d_Bh, int32_t ldb, int32_t b_dtype,
                                float* d_C, int32_t N, ra_stream_t stream) {
    if (!p) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: plan is NULL");
    if (!p->info.active)
        return ra::fail(RA_ERR_INACTIVE_PLAN, "tile: plan is inactive (built with N < 16 or empty matrix)");
    if (N <= 0 || p->info.M == 0) return RA_OK;
    if (!d_Bh || !d_C) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: NULL B or C");
    if (ldb < N || (ldb % 8) != 0 || !ra::aligned16(d_Bh))
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: low-precision B needs ldb >= N, ldb % 8 == 0, 16-byte alignment");
    const bool bf16 = b_dtype == RA_DTYPE_BF16;
    if (b_dtype != RA_DTYPE_F16 && !bf16) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: b_dtype must be F16 or BF16");
    if (bf16 != (p->info.value_dtype == RA_DTYPE_BF16))
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: B precision differs from the plan's value dtype");
    return run_common(p, static_cast<const uint16_t*>(d_Bh), ldb, bf16, d_C, N, reinterpret_cast<hipStream_t>(stream));
}

ra_status ra_tile_plan_get_info(const ra_tile_plan* p, ra_tile_info* info) {
    if (!p || !info) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: NULL argument");
    *info = p->info;
    return RA_OK;
}

void ra_tile_plan_destroy(ra_tile_plan* p) { delete p; }

}  // extern "C"
