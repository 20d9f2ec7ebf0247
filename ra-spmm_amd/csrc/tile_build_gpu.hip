// tile_build_gpu.hip — device build of the tile format (cold path).
//
// Same windows, vectors, blocks, value rounding and segment tables as the host
// builder (tile_build.cpp), produced with sorts and scans on the GPU:
//   1. (COMMUNITY_TC) rows sorted by (leading column or INT_MAX, row) -> window slots
//   2. the row of every nonzero (row starts marked, then a max-scan) and one
//      64-bit key per nonzero: (cell << (cb + log2 rows)) | (column << log2 rows) | slot,
//      cb = bits of K - 1 (the fewer key bits, the fewer radix passes)
//   3. stable radix sort of (key, value)  -> per-window (col, slot) order,
//      duplicates adjacent in CSR order, values in key order
//   4. scans: vector ids, vectors and blocks per window, block offsets
//   5. scatter: atox (first entry of each vector), values (first entry of each
//      (col, slot) sums its duplicates in CSR order, scales, rounds)
//   6. segment tables of the split schedule (64 blocks for SEGMENT_HYBRID,
//      kTileDirectSplitBlocks otherwise)
// Reference algorithm: tc/ra_tc_direct.cu:654-706, tc/ra_community_tc.cu:335-403,
// tc/ra_segment_hybrid.cu:470-498 (the reference builds on the host with OpenMP).
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <cstdlib>

#include "half_convert.hpp"
#include "ra_internal.hpp"
#include "tile_format.hpp"

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 20)));
}

#define RA_GRID_STRIDE(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

__global__ void fill_i32(int32_t* p, int64_t n, int32_t v) { RA_GRID_STRIDE(i, n) p[i] = v; }
__global__ void fill_u16(uint16_t* p, int64_t n) { RA_GRID_STRIDE(i, n) p[i] = 0; }
__global__ void fill_u32(unsigned* p, int64_t n) { RA_GRID_STRIDE(i, n) p[i] = 0u; }

// Validity counters: [0] rows with rowptr[r+1] < rowptr[r], [1] columns outside [0, K).
__global__ void validate_csr(const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colind,
                             int M, int K, int64_t base, int64_t n, unsigned* __restrict__ bad) {
    RA_GRID_STRIDE(r, (int64_t)M) {
        if (rowptr[r + 1] < rowptr[r]) atomicAdd(&bad[0], 1u);
    }
    RA_GRID_STRIDE(t, n) {
        const int c = colind[base + t];
        if (c < 0 || c >= K) atomicAdd(&bad[1], 1u);
    }
}

// max |v| as the bit pattern of a non-negative float (monotone as unsigned):
// wave, then workgroup reduction through LDS, one atomic per workgroup (the
// launch is capped at kReduceBlocks workgroups).
constexpr int kReduceBlocks = 1024;
__global__ void abs_max_bits(const float* __restrict__ vals, int64_t base, int64_t n,
                             unsigned* __restrict__ out) {
    __shared__ unsigned part[kThreads / 64];
    unsigned m = 0;
    RA_GRID_STRIDE(t, n) {
        const unsigned b = ra::float_bits(vals[base + t]) & 0x7FFFFFFFu;
        if (b <= 0x7F800000u) m = max(m, b);  // ignore NaN payloads
    }
    for (int off = 32; off > 0; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < kThreads / 64; ++i) m = max(m, part[i]);
        atomicMax(out, m);
    }
}

__global__ void lead_keys(const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colind, int M,
                          uint64_t* __restrict__ keys) {
    RA_GRID_STRIDE(r, (int64_t)M) {
        const uint32_t lead = rowptr[r] < rowptr[r + 1] ? static_cast<uint32_t>(colind[rowptr[r]])
                                                        : static_cast<uint32_t>(INT_MAX);
        keys[r] = (static_cast<uint64_t>(lead) << 32) | static_cast<uint32_t>(r);
    }
}

// Sorted leading-column order: order[i] = row at position i, pos[row] = i.
__global__ void place_rows(const uint64_t* __restrict__ sorted, int M, int32_t* __restrict__ order,
                           int32_t* __restrict__ pos) {
    RA_GRID_STRIDE(i, (int64_t)M) {
        const int32_t row = static_cast<int32_t>(sorted[i] & 0xFFFFFFFFu);
        order[i] = row;
        pos[row] = static_cast<int32_t>(i);
    }
}

// win_rows[slot] = row at that position (identity without an order), -1 pad.
__global__ void fill_win_rows(const int32_t* __restrict__ order, int M, int64_t slots,
                              int32_t* __restrict__ win_rows) {
    RA_GRID_STRIDE(i, slots) {
        win_rows[i] = i < M ? (order ? order[i] : static_cast<int32_t>(i)) : -1;
    }
}

// Window geometry: 2^sb rows per window, vb vectors per block.  sb = 3, vb = 8
// is the reference's 8-row format; sb = 4 or 5 with vb = 32 is the tall format
// (16 or 32 rows, one MFMA K of vectors per block).
struct Layout {
    int sb;
    int vb;
    int cb;  // column bits of the sort key
};

// Row of every nonzero position: each non-empty row marks its first position,
// then an inclusive max-scan carries it over the row (rows ascend with
// position).  Two streaming passes instead of a binary search per nonzero
// (18 dependent loads each on C4).
__global__ void mark_row_starts(const int32_t* __restrict__ rowptr, int M, int64_t base,
                                int32_t* __restrict__ row_of) {
    RA_GRID_STRIDE(r, (int64_t)M) {
        if (rowptr[r + 1] > rowptr[r]) row_of[rowptr[r] - base] = static_cast<int32_t>(r);
    }
}

// Key of every nonzero: (window << (cb + sb)) | (column << sb) | slot.
// With column partitions the "window" of a key is the cell
// part * W + window, part = column / cols_per_part (partition-major cells).
// vout (when given) receives each nonzero's value, so that the key sort
// carries the values along and the scatter reads them in key order.
__global__ void entry_keys(const int32_t* __restrict__ row_of, const int32_t* __restrict__ colind,
                           const float* __restrict__ vals, const int32_t* __restrict__ pos, int64_t base, int64_t n,
                           int sb, int cb, int cols_per_part, int64_t W, uint64_t* __restrict__ keys,
                           float* __restrict__ vout) {
    RA_GRID_STRIDE(t, n) {
        const int64_t p = base + t;
        const int lo = row_of[t];
        const int64_t slot_pos = pos ? pos[lo] : lo;
        const int64_t cell = (int64_t)(colind[p] / cols_per_part) * W + (slot_pos >> sb);
        keys[t] = (static_cast<uint64_t>(cell) << (cb + sb)) |
                  (static_cast<uint64_t>(static_cast<uint32_t>(colind[p])) << sb) |
                  static_cast<uint64_t>(slot_pos & ((1 << sb) - 1));
        if (vout) vout[t] = vals[p];
    }
}

// Window-height sampling: flag[t] = 1 when nonzero t lies in a sampled
// 32-row window (every S-th), and the sampled keys (32-row windows, sb = 5)
// written compactly at the exclusive-scan offsets of the flags.
__global__ void sample_flags(const int32_t* __restrict__ row_of, const int32_t* __restrict__ pos, int64_t n, int S,
                             int32_t* __restrict__ flag) {
    RA_GRID_STRIDE(t, n) {
        const int lo = row_of[t];
        const int64_t slot_pos = pos ? pos[lo] : lo;
        flag[t] = ((slot_pos >> 5) % S) == 0 ? 1 : 0;
    }
}

__global__ void sampled_keys(const int32_t* __restrict__ row_of, const int32_t* __restrict__ colind,
                             const int32_t* __restrict__ pos, int64_t base, int64_t n, int cb, int S,
                             const int32_t* __restrict__ off, uint64_t* __restrict__ keys) {
    RA_GRID_STRIDE(t, n) {
        const int lo = row_of[t];
        const int64_t slot_pos = pos ? pos[lo] : lo;
        const int64_t w = slot_pos >> 5;
        if (w % S != 0) continue;
        keys[off[t]] = (static_cast<uint64_t>(w) << (cb + 5)) |
                       (static_cast<uint64_t>(static_cast<uint32_t>(colind[base + t])) << 5) |
                       static_cast<uint64_t>(slot_pos & 31);
    }
}

__global__ void mark_new(const uint64_t* __restrict__ keys, int64_t n, int sb, int32_t* __restrict__ newvec,
                         int32_t* __restrict__ newkey) {
    RA_GRID_STRIDE(i, n) {
        const uint64_t k = keys[i];
        const bool first = i == 0;
        const uint64_t prev = first ? 0 : keys[i - 1];
        newvec[i] = (first || (k >> sb) != (prev >> sb)) ? 1 : 0;
        newkey[i] = (first || k != prev) ? 1 : 0;
    }
}

// Distinct (row / h, column) pairs for h = 8, 16, 32 from keys sorted at
// sb = 5: within a (32-row window, column) run the slots ascend, so a new
// h-window starts where slot >> log2(h) changes.
__global__ void count_layouts(const uint64_t* __restrict__ keys, int64_t n, unsigned long long* __restrict__ out) {
    __shared__ unsigned long long part[3][kThreads / 64];
    unsigned long long c[3] = {0, 0, 0};
    RA_GRID_STRIDE(i, n) {
        const uint64_t k = keys[i];
        const bool first = i == 0 || (keys[i - 1] >> 5) != (k >> 5);
        const uint64_t prev = i == 0 ? 0 : keys[i - 1];
        c[0] += first || ((prev & 31) >> 3) != ((k & 31) >> 3);
        c[1] += first || ((prev & 31) >> 4) != ((k & 31) >> 4);
        c[2] += first;
    }
    for (int t = 0; t < 3; ++t) {
        unsigned long long v = c[t];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if ((threadIdx.x & 63) == 0) part[t][threadIdx.x >> 6] = v;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
        unsigned long long v = 0;
        for (int i = 0; i < kThreads / 64; ++i) v += part[threadIdx.x][i];
        atomicAdd(&out[threadIdx.x], v);
    }
}

// Vectors are numbered in (window, column) order, so the last vector id of a
// window's entries is the number of vectors in windows <= w.  Windows without
// entries keep 0 and get the running value from a max-scan.
__global__ void window_last_vid(const uint64_t* __restrict__ keys, const int32_t* __restrict__ vid, int64_t n,
                                int wshift, int32_t* __restrict__ last) {
    RA_GRID_STRIDE(i, n) {
        const uint64_t w = keys[i] >> wshift;
        if (i == n - 1 || (keys[i + 1] >> wshift) != w) last[w] = vid[i];
    }
}

__global__ void vectors_from_cum(const int32_t* __restrict__ cum, int W, int32_t* __restrict__ nvec) {
    RA_GRID_STRIDE(w, (int64_t)W) nvec[w] = cum[w] - (w > 0 ? cum[w - 1] : 0);
}

__global__ void window_counts(const int32_t* __restrict__ nvec, int W, int vb, int limit,
                              int32_t* __restrict__ blocks, int32_t* __restrict__ segs,
                              int32_t* __restrict__ split_slots, int32_t* __restrict__ is_split) {
    RA_GRID_STRIDE(w, (int64_t)W) {
        const int b = (nvec[w] + vb - 1) / vb;
        blocks[w] = b;
        const bool split = b > limit;
        const int ns = split ? (b + limit - 1) / limit : 1;
        segs[w] = ns;
        split_slots[w] = split ? ns : 0;
        is_split[w] = split ? 1 : 0;
    }
}

__global__ void scatter_entries(const uint64_t* __restrict__ keys, const float* __restrict__ svals,
                                const int32_t* __restrict__ vid, const int32_t* __restrict__ newkey, int64_t n,
                                const int32_t* __restrict__ block_offsets,
                                const int32_t* __restrict__ win_vec_start, float vscale, int bf16, Layout L,
                                int32_t* __restrict__ atox, uint16_t* __restrict__ out) {
    const int rows = 1 << L.sb;
    RA_GRID_STRIDE(i, n) {
        if (!newkey[i]) continue;
        const uint64_t k = keys[i];
        const int64_t w = static_cast<int64_t>(k >> (L.cb + L.sb));
        const int32_t col = static_cast<int32_t>((k >> L.sb) & ((uint64_t(1) << L.cb) - 1));
        const int slot = static_cast<int>(k & static_cast<uint64_t>(rows - 1));
        const int64_t vlocal = (int64_t)(vid[i] - 1) - win_vec_start[w];
        const int64_t blk = block_offsets[w] + vlocal / L.vb;
        const int kk = static_cast<int>(vlocal % L.vb);
        atox[blk * L.vb + kk] = col;
        // Duplicates of (window, col, slot) follow in CSR order (stable sort).
        float acc = 0.f + svals[i];
        for (int64_t j = i + 1; j < n && keys[j] == k; ++j) acc += svals[j];
        // 8-row blocks: [slot][vector]; tall blocks: [slot/16][vector/8][slot%16][vector%8],
        // the 16-byte run one MFMA lane (row slot%16, K group vector/8) loads.
        const int64_t at = L.vb == 8 ? blk * 64 + slot * 8 + kk
                                     : blk * ((int64_t)rows * 32) +
                                           ((((slot >> 4) * 4 + (kk >> 3)) * 16 + (slot & 15)) * 8 + (kk & 7));
        out[at] = bf16 ? ra::bf16_rne_bits(acc) : ra::half_rne_bits(acc * vscale);
    }
}

__global__ void fill_segments(const int32_t* __restrict__ block_offsets, const int32_t* __restrict__ seg_start,
                              const int32_t* __restrict__ slot_start, const int32_t* __restrict__ split_idx,
                              int W, int limit, int32_t* __restrict__ seg_window,
                              int32_t* __restrict__ seg_bbegin, int32_t* __restrict__ seg_bend,
                              int32_t* __restrict__ seg_slot, int32_t* __restrict__ split_windows,
                              int32_t* __restrict__ split_offsets) {
    RA_GRID_STRIDE(w, (int64_t)W) {
        const int b0 = block_offsets[w], b1 = block_offsets[w + 1];
        const int s0 = seg_start[w];
        if (b1 - b0 <= limit) {
            seg_window[s0] = static_cast<int32_t>(static_cast<uint32_t>(w) | ra::kTileSoleFlag);
            seg_bbegin[s0] = b0;
            seg_bend[s0] = b1;
            seg_slot[s0] = -1;
        } else {
            int t = 0;
            for (int b = b0; b < b1; b += limit, ++t) {
                seg_window[s0 + t] = static_cast<int32_t>(w);
                seg_bbegin[s0 + t] = b;
                seg_bend[s0 + t] = min(b + limit, b1);
                seg_slot[s0 + t] = slot_start[w] + t;
            }
            const int j = split_idx[w];
            split_windows[j] = static_cast<int32_t>(w);
            split_offsets[j + 1] = slot_start[w] + t;
        }
        if (w == 0) split_offsets[0] = 0;
    }
}

struct Scratch {
    ra::DeviceBuffer buf;
    template <typename T>
    T* take(size_t count, size_t& off) {
        off = (off + 255) & ~size_t(255);
        T* p = reinterpret_cast<T*>(buf.get<char>() + off);
        off += count * sizeof(T);
        return p;
    }
};

template <typename T>
ra_status read_back(T* dst, const T* src, size_t n, hipStream_t st) {
    RA_HIP_TRY(hipMemcpyAsync(dst, src, n * sizeof(T), hipMemcpyDeviceToHost, st));
    RA_HIP_TRY(hipStreamSynchronize(st));
    return RA_OK;
}

// Window height for rows_per_window = 0, from the distinct (row / h, column)
// counts v8, v16, v32.  Cost model: vector-memory instructions per 32 vectors
// (8 B-row gathers and the index load, plus the A loads: one per 16 rows of a
// tall block, one per 4 blocks of the 8-row format), so 10 per 32 vectors for
// h = 8 and 16 and 11 for h = 32.  A tall layout is taken only when the model
// saves at least 15%: measured on MI355X, the 32-row kernel runs C3 (SBM,
// N=256) in 0.61 ms against 0.69 ms with 8 rows (model: -30%), and graphs whose
// rows share few columns (C2, C4, C5) run 2-15% slower with 16 or 32 rows.
// Tall blocks hold h*32 values; a height whose values would pass 2^31 is skipped.
int choose_rows(unsigned long long v8, unsigned long long v16, unsigned long long v32, int64_t M) {
    const double c8 = 10.0 * v8, c16 = 10.0 * v16, c32 = 11.0 * v32;
    auto fits = [&](int h, unsigned long long v) {
        const double blocks = static_cast<double>(v) / 32.0 + static_cast<double>((M + h - 1) / h);
        return blocks * h * 32.0 < static_cast<double>(INT32_MAX);
    };
    if (c32 <= 0.85 * c8 && c32 <= c16 && fits(32, v32)) return 32;
    if (c16 <= 0.85 * c8 && fits(16, v16)) return 16;
    return 8;
}

ra_status gpu_build(ra_tile_plan* p, int32_t kind, const int32_t* rowptr, const int32_t* colind,
                    const float* vals, int32_t M, int32_t K, int32_t N, int32_t value_dtype, int32_t rows_req,
                    hipStream_t st) {
    p->info = ra_tile_info{};
    p->info.kind = kind;
    p->info.M = M;
    p->info.K = K;
    p->info.value_dtype = value_dtype;
    p->info.rows_per_window = rows_req > 0 ? rows_req : ra::kTileWindow;
    p->info.col_parts = 1;
    if (M == 0 || K == 0 || N < 16) return RA_OK;  // inactive, like the host build
    int32_t ends[2];
    RA_TRY(read_back(&ends[0], rowptr, 1, st));
    RA_TRY(read_back(&ends[1], rowptr + M, 1, st));
    const int64_t base = ends[0];
    const int64_t n = static_cast<int64_t>(ends[1]) - ends[0];
    if (n < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: rowptr not monotone");
    if (n > INT32_MAX) return ra::fail(RA_ERR_UNSUPPORTED, "tile: more than 2^31-1 nonzeros");
    if (n > 0 && (!colind || !vals)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: colind/vals NULL");
    // Column partitions: P > 1 cuts every window into P cells by column range
    // (partition-major), so that the kernels can run one partition at a time
    // and keep the gathered working set (K / P rows of B) near the L2 size.
    // Auto: P = 8 for long rows (nnz / M >= 128) over wide B (K >= 65536),
    // where the per-partition accumulation into C costs little against the
    // gathers; RA_TILE_COL_PARTS fixes it (1, 2, 4, 8 or 16).
    int P = (K >= 65536 && n >= 128LL * M) ? 8 : 1;
    if (const char* e = std::getenv("RA_TILE_COL_PARTS")) {
        const int v = std::atoi(e);
        if (v == 1 || v == 2 || v == 4 || v == 8 || v == 16) P = v;
    }
    const int cols_per_part = static_cast<int>((static_cast<int64_t>(K) + P - 1) / P);
    int cb = 1;  // column bits of the sort keys: columns are < K <= 2^cb
    while ((int64_t(1) << cb) < K) ++cb;
    const int64_t Wmax = (M + ra::kTileWindow - 1) / ra::kTileWindow * P;  // most cells of any layout
    const bool bf16 = value_dtype == RA_DTYPE_BF16;
    const int64_t nn = std::max<int64_t>(n, 1);

    // Temporary storage for the sorts and scans, sized by a dry run.
    size_t sort_bytes = 0, scan_bytes = 0, red_bytes = 0;
    uint64_t* knull = nullptr;
    int32_t* inull = nullptr;
    float* fnull = nullptr;
    RA_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, knull, knull, fnull, fnull,
                                                  static_cast<int>(std::max<int64_t>(nn, M)), 0, 64, st));
    RA_HIP_TRY(hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, inull, inull, static_cast<int>(nn), st));
    size_t scan2 = 0;
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, scan2, inull, inull, static_cast<int>(Wmax + 1), st));
    scan_bytes = std::max(scan_bytes, scan2);
    RA_HIP_TRY(hipcub::DeviceReduce::Max(nullptr, red_bytes, inull, inull, static_cast<int>(Wmax), st));
    size_t scan3 = 0;
    RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(nullptr, scan3, inull, inull, hipcub::Max(),
                                                 static_cast<int>(Wmax), st));
    scan_bytes = std::max(scan_bytes, scan3);
    size_t red2 = 0;
    RA_HIP_TRY(hipcub::DeviceReduce::Sum(nullptr, red2, inull, inull, static_cast<int>(nn), st));
    red_bytes = std::max(red_bytes, red2);
    size_t scan5 = 0;
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, scan5, inull, inull, static_cast<int>(nn), st));
    scan_bytes = std::max(scan_bytes, scan5);
    size_t scan4 = 0;
    RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(nullptr, scan4, inull, inull, hipcub::Max(), static_cast<int>(nn),
                                                 st));
    scan_bytes = std::max(scan_bytes, scan4);
    const size_t tmp_bytes = std::max({sort_bytes, scan_bytes, red_bytes});

    const size_t need = 256 * 27 + tmp_bytes + nn * (2 * 8 + 2 * 4 + 4 * 4) +
                        std::max<int64_t>(M, 1) * (2 * 8 + 4 + 4) + (Wmax + 1) * 4 * 9 + 64;
    Scratch s;
    RA_TRY(s.buf.allocate(need));
    size_t off = 0;
    void* tmp = s.take<char>(tmp_bytes, off);
    uint64_t* keys = s.take<uint64_t>(nn, off);
    uint64_t* keys2 = s.take<uint64_t>(nn, off);
    float* fval = s.take<float>(nn, off);   // values in CSR order, then sorted with the keys
    float* fval2 = s.take<float>(nn, off);
    int32_t* newvec = s.take<int32_t>(nn, off);
    int32_t* newkey = s.take<int32_t>(nn, off);
    int32_t* vid = s.take<int32_t>(nn, off);
    int32_t* row_of = s.take<int32_t>(nn, off);
    uint64_t* rkeys = s.take<uint64_t>(std::max<int64_t>(M, 1), off);
    uint64_t* rkeys2 = s.take<uint64_t>(std::max<int64_t>(M, 1), off);
    int32_t* pos = s.take<int32_t>(std::max<int64_t>(M, 1), off);
    int32_t* order = s.take<int32_t>(std::max<int64_t>(M, 1), off);
    int32_t* nvec = s.take<int32_t>(Wmax + 1, off);
    int32_t* wvec_start = s.take<int32_t>(Wmax + 1, off);
    int32_t* blocks = s.take<int32_t>(Wmax + 1, off);
    int32_t* segs = s.take<int32_t>(Wmax + 1, off);
    int32_t* seg_start = s.take<int32_t>(Wmax + 1, off);
    int32_t* split_slots = s.take<int32_t>(Wmax + 1, off);
    int32_t* slot_start = s.take<int32_t>(Wmax + 1, off);
    int32_t* is_split = s.take<int32_t>(Wmax + 1, off);
    int32_t* split_idx = s.take<int32_t>(Wmax + 1, off);
    unsigned* flags = s.take<unsigned>(4, off);
    int32_t* red_out = s.take<int32_t>(2, off);
    unsigned long long* layout_counts = s.take<unsigned long long>(3, off);

    // Validation and value scale.
    fill_u32<<<1, kThreads, 0, st>>>(flags, 4);
    validate_csr<<<grid_for(std::max<int64_t>(M, n)), kThreads, 0, st>>>(rowptr, colind, M, K, base, n, flags);
    abs_max_bits<<<std::min<unsigned>(grid_for(n), kReduceBlocks), kThreads, 0, st>>>(vals, base, n, flags + 2);
    RA_LAUNCH_CHECK("validate_csr");
    unsigned hflags[4];
    RA_TRY(read_back(hflags, flags, 4, st));
    if (hflags[0]) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: rowptr not monotone");
    if (hflags[1]) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: column index out of range");
    float vmax;
    std::memcpy(&vmax, &hflags[2], 4);
    p->info.value_scale_log2 = bf16 ? 0 : ra::f16_value_scale_log2(vmax);
    const float vscale = std::ldexp(1.0f, p->info.value_scale_log2);

    // Row of every nonzero (rowptr is monotone by now): marks in `newvec`,
    // which mark_new overwrites later, max-scanned into row_of.
    if (n > 0) {
        fill_i32<<<grid_for(n), kThreads, 0, st>>>(newvec, n, 0);
        mark_row_starts<<<grid_for(M), kThreads, 0, st>>>(rowptr, M, base, newvec);
        size_t tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(tmp, tb, newvec, row_of, hipcub::Max(), static_cast<int>(n), st));
        RA_LAUNCH_CHECK("row ids");
    }

    // Row order: COMMUNITY_TC sorts rows by leading column (ties by row).
    const int32_t* pos_ptr = nullptr;
    const int32_t* order_ptr = nullptr;
    if (kind == RA_TILE_COMMUNITY_TC) {
        lead_keys<<<grid_for(M), kThreads, 0, st>>>(rowptr, colind, M, rkeys);
        // Keys are unique, so the radix sort yields the stable leading-column order.
        size_t tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceRadixSort::SortKeys(tmp, tb, rkeys, rkeys2, M, 0, 63, st));
        place_rows<<<grid_for(M), kThreads, 0, st>>>(rkeys2, M, order, pos);
        pos_ptr = pos;
        order_ptr = order;
    }
    RA_LAUNCH_CHECK("row order");

    // Window height: asked for, or the cheapest by the address-unit model from
    // the distinct (row / h, column) counts of one sort at h = 32.
    int rows = rows_req;
    if (rows == 0) {
        // RA_TILE_ROWS=8|16|32 fixes the automatic choice (measurement runs).
        if (const char* e = std::getenv("RA_TILE_ROWS")) rows = std::atoi(e);
    }
    if (rows == 0) {
        rows = ra::kTileWindow;
        if (n > 0) {
            // Counts from every S-th 32-row window (S a power of two <= 16,
            // at least 2^21 sampled nonzeros and 512 sampled windows): the
            // counts estimate the full ones up to the factor S, and sorting
            // 1/S of the keys costs 1/S of the sort.  Deterministic.
            const int64_t W32 = (M + 31) / 32;
            int S = 1;
            while (S < 16 && n / (2 * S) >= (int64_t(1) << 21) && W32 / (2 * S) >= 512) S *= 2;
            int64_t ns = n;
            fill_u32<<<1, kThreads, 0, st>>>(reinterpret_cast<unsigned*>(layout_counts), 6);
            if (S == 1) {
                entry_keys<<<grid_for(n), kThreads, 0, st>>>(row_of, colind, vals, pos_ptr, base, n, 5, cb, INT32_MAX,
                                                             W32, keys, nullptr);
            } else {
                sample_flags<<<grid_for(n), kThreads, 0, st>>>(row_of, pos_ptr, n, S, newvec);
                size_t tb = tmp_bytes;
                RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, newvec, vid, static_cast<int>(n), st));
                sampled_keys<<<grid_for(n), kThreads, 0, st>>>(row_of, colind, pos_ptr, base, n, cb, S, vid, keys);
                int32_t last[2];
                RA_TRY(read_back(&last[0], vid + n - 1, 1, st));
                RA_TRY(read_back(&last[1], newvec + n - 1, 1, st));
                ns = static_cast<int64_t>(last[0]) + last[1];
            }
            RA_LAUNCH_CHECK("height sample keys");
            int wb = 0;
            while ((int64_t(1) << wb) < W32) ++wb;
            if (ns > 0) {
                size_t tb = tmp_bytes;
                RA_HIP_TRY(hipcub::DeviceRadixSort::SortKeys(tmp, tb, keys, keys2, static_cast<int>(ns), 0,
                                                             5 + cb + wb, st));
                count_layouts<<<std::min<unsigned>(grid_for(ns), kReduceBlocks), kThreads, 0, st>>>(keys2, ns,
                                                                                                     layout_counts);
                RA_LAUNCH_CHECK("count_layouts");
            }
            unsigned long long v[3];
            RA_TRY(read_back(v, layout_counts, 3, st));
            rows = choose_rows(v[0] * S, v[1] * S, v[2] * S, M);
        }
    }
    if (rows != 8 && rows != 16 && rows != 32)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: rows per window must be 8, 16 or 32");
    const Layout L{rows == 8 ? 3 : rows == 16 ? 4 : 5, rows == 8 ? 8 : 32, cb};
    const int64_t W = (M + rows - 1) / rows;
    const int64_t slots = W * rows;
    // Split limits in vectors: 64 8-vector blocks for SEGMENT_HYBRID (the
    // reference rule), kTileDirectSplitBlocks of them for the other kinds.
    const int limit =
        (kind == RA_TILE_SEGMENT_HYBRID ? ra::kTileSegBlocks : ra::kTileDirectSplitBlocks) * ra::kTileVec / L.vb;
    p->info.rows_per_window = rows;
    RA_TRY(p->win_rows.allocate(slots * sizeof(int32_t)));
    fill_win_rows<<<grid_for(slots), kThreads, 0, st>>>(order_ptr, M, slots, p->win_rows.get<int32_t>());
    RA_LAUNCH_CHECK("window slots");

    // Sort nonzeros by (cell, column, slot), stable in CSR position.
    const int64_t NC = W * P;
    if (NC >= INT32_MAX)
        return ra::fail(RA_ERR_UNSUPPORTED, "tile: too many windows x column partitions for int32 cell ids");
    int wbits = 0;
    while ((int64_t(1) << wbits) < NC) ++wbits;
    const int wshift = L.cb + L.sb;
    if (wshift + wbits > 64) return ra::fail(RA_ERR_UNSUPPORTED, "tile: sort key wider than 64 bits");
    if (n > 0) {
        entry_keys<<<grid_for(n), kThreads, 0, st>>>(row_of, colind, vals, pos_ptr, base, n, L.sb, L.cb,
                                                     cols_per_part, W, keys, fval);
        size_t tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(tmp, tb, keys, keys2, fval, fval2, static_cast<int>(n),
                                                      0, wshift + wbits, st));
        mark_new<<<grid_for(n), kThreads, 0, st>>>(keys2, n, L.sb, newvec, newkey);
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::InclusiveSum(tmp, tb, newvec, vid, static_cast<int>(n), st));
    }
    // nvec[w] from the last vector id of each window (no atomics): wvec_start
    // is used as the temporary for the per-window last ids and their max-scan.
    fill_i32<<<grid_for(NC + 1), kThreads, 0, st>>>(nvec, NC + 1, 0);
    fill_i32<<<grid_for(NC + 1), kThreads, 0, st>>>(wvec_start, NC + 1, 0);
    if (n > 0) {
        window_last_vid<<<grid_for(n), kThreads, 0, st>>>(keys2, vid, n, wshift, wvec_start);
        size_t tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(tmp, tb, wvec_start, nvec, hipcub::Max(), static_cast<int>(NC), st));
        vectors_from_cum<<<grid_for(NC), kThreads, 0, st>>>(nvec, static_cast<int>(NC), wvec_start);
        RA_HIP_TRY(hipMemcpyAsync(nvec, wvec_start, NC * sizeof(int32_t), hipMemcpyDeviceToDevice, st));
    }
    window_counts<<<grid_for(NC), kThreads, 0, st>>>(nvec, static_cast<int>(NC), L.vb, limit, blocks, segs,
                                                    split_slots, is_split);
    fill_i32<<<1, kThreads, 0, st>>>(blocks + NC, 1, 0);
    fill_i32<<<1, kThreads, 0, st>>>(segs + NC, 1, 0);
    fill_i32<<<1, kThreads, 0, st>>>(split_slots + NC, 1, 0);
    fill_i32<<<1, kThreads, 0, st>>>(is_split + NC, 1, 0);
    RA_LAUNCH_CHECK("window counts");
    RA_TRY(p->block_offsets.allocate((NC + 1) * sizeof(int32_t)));
    int32_t* boff = p->block_offsets.get<int32_t>();
    {
        size_t tb = tmp_bytes;
        const int wn = static_cast<int>(NC + 1);
        RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, nvec, wvec_start, wn, st));
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, blocks, boff, wn, st));
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, segs, seg_start, wn, st));
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, split_slots, slot_start, wn, st));
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp, tb, is_split, split_idx, wn, st));
        tb = tmp_bytes;
        RA_HIP_TRY(hipcub::DeviceReduce::Max(tmp, tb, blocks, red_out, static_cast<int>(NC), st));
        if (n > 0) {
            tb = tmp_bytes;
            RA_HIP_TRY(hipcub::DeviceReduce::Sum(tmp, tb, newkey, red_out + 1, static_cast<int>(n), st));
        } else {
            fill_i32<<<1, kThreads, 0, st>>>(red_out + 1, 1, 0);
        }
    }
    int32_t totals[6];  // blocks, vectors, segments, slots, split windows
    RA_TRY(read_back(&totals[0], boff + NC, 1, st));
    RA_TRY(read_back(&totals[1], wvec_start + NC, 1, st));
    RA_TRY(read_back(&totals[2], seg_start + NC, 1, st));
    RA_TRY(read_back(&totals[3], slot_start + NC, 1, st));
    RA_TRY(read_back(&totals[4], split_idx + NC, 1, st));
    int32_t reds[2];
    RA_TRY(read_back(reds, red_out, 2, st));
    const int64_t nblocks = totals[0];
    const int64_t block_vals = (int64_t)rows * L.vb;  // values per block
    if (nblocks * block_vals > INT32_MAX) return ra::fail(RA_ERR_UNSUPPORTED, "tile: too many blocks for int32 offsets");

    // atox, values.
    RA_TRY(p->atox.allocate(std::max<int64_t>(nblocks, 1) * L.vb * sizeof(int32_t)));
    RA_TRY(p->vals.allocate(std::max<int64_t>(nblocks, 1) * block_vals * sizeof(uint16_t)));
    fill_i32<<<grid_for(nblocks * L.vb), kThreads, 0, st>>>(p->atox.get<int32_t>(), nblocks * L.vb, -1);
    fill_u16<<<grid_for(nblocks * block_vals), kThreads, 0, st>>>(p->vals.get<uint16_t>(), nblocks * block_vals);
    if (n > 0)
        scatter_entries<<<grid_for(n), kThreads, 0, st>>>(keys2, fval2, vid, newkey, n, boff,
                                                          wvec_start, vscale, bf16 ? 1 : 0, L,
                                                          p->atox.get<int32_t>(), p->vals.get<uint16_t>());
    RA_LAUNCH_CHECK("scatter_entries");

    // Segment tables.
    const int64_t nseg = totals[2], nsplit = totals[4];
    RA_TRY(p->seg_window.allocate(nseg * sizeof(int32_t)));
    RA_TRY(p->seg_bbegin.allocate(nseg * sizeof(int32_t)));
    RA_TRY(p->seg_bend.allocate(nseg * sizeof(int32_t)));
    RA_TRY(p->seg_slot.allocate(nseg * sizeof(int32_t)));
    RA_TRY(p->split_windows.allocate(std::max<int64_t>(nsplit, 1) * sizeof(int32_t)));
    RA_TRY(p->split_offsets.allocate((nsplit + 1) * sizeof(int32_t)));
    fill_segments<<<grid_for(NC), kThreads, 0, st>>>(boff, seg_start, slot_start, split_idx, static_cast<int>(NC),
                                                    limit, p->seg_window.get<int32_t>(), p->seg_bbegin.get<int32_t>(),
                                                    p->seg_bend.get<int32_t>(), p->seg_slot.get<int32_t>(),
                                                    p->split_windows.get<int32_t>(), p->split_offsets.get<int32_t>());
    RA_LAUNCH_CHECK("fill_segments");
    RA_HIP_TRY(hipStreamSynchronize(st));

    // First segment and first split window of every partition (cells are
    // partition-major, so each partition's items are one contiguous run).
    p->part_items.assign(P + 1, 0);
    p->part_splits.assign(P + 1, 0);
    for (int q = 1; q <= P; ++q) {
        RA_TRY(read_back(&p->part_items[q], seg_start + (int64_t)q * W, 1, st));
        RA_TRY(read_back(&p->part_splits[q], split_idx + (int64_t)q * W, 1, st));
    }

    ra_tile_info& I = p->info;
    I.active = 1;
    I.col_parts = P;
    I.num_windows = static_cast<int32_t>(W);
    I.num_blocks = static_cast<int32_t>(nblocks);
    I.num_segments = static_cast<int32_t>(nseg);
    I.num_split_windows = static_cast<int32_t>(nsplit);
    I.num_split_segs = totals[3];
    I.max_window_blocks = reds[0];
    I.nnz = reds[1];
    I.num_vectors = totals[1];
    I.avg_tile_density =
        nblocks > 0 ? static_cast<float>(static_cast<double>(I.nnz) / (static_cast<double>(block_vals) * nblocks)) : 0.f;
    I.plan_bytes = static_cast<int64_t>(4 * (slots + (W * P + 1) + nblocks * L.vb + 4 * nseg + nsplit + nsplit + 1) +
                                        2 * nblocks * block_vals);
    p->num_items = static_cast<int32_t>(nseg);
    return RA_OK;
}

const ra::DeviceBuffer* plan_array(const ra_tile_plan* p, const std::string& n, size_t& elem, int64_t& count) {
    const ra_tile_info& I = p->info;
    const int64_t W = I.num_windows;
    elem = 4;
    if (n == "block_offsets") { count = I.active ? W * std::max(I.col_parts, 1) + 1 : 0; return &p->block_offsets; }
    const int64_t rows = I.rows_per_window > 0 ? I.rows_per_window : ra::kTileWindow;
    const int64_t vb = rows == ra::kTileWindow ? ra::kTileVec : 32;
    if (n == "atox") { count = (int64_t)I.num_blocks * vb; return &p->atox; }
    if (n == "win_rows") { count = W * rows; return &p->win_rows; }
    if (n == "vals") { elem = 2; count = (int64_t)I.num_blocks * rows * vb; return &p->vals; }
    if (n == "seg_window") { count = I.num_segments; return &p->seg_window; }
    if (n == "seg_bbegin") { count = I.num_segments; return &p->seg_bbegin; }
    if (n == "seg_bend") { count = I.num_segments; return &p->seg_bend; }
    if (n == "seg_slot") { count = I.num_segments; return &p->seg_slot; }
    if (n == "split_windows") { count = I.num_split_windows; return &p->split_windows; }
    if (n == "split_offsets") { count = I.active ? I.num_split_windows + 1 : 0; return &p->split_offsets; }
    return nullptr;
}

}  // namespace

extern "C" {

ra_status ra_tile_plan_create_device(int32_t kind, const int32_t* d_rowptr, const int32_t* d_colind,
                                     const float* d_vals, int32_t M, int32_t K, int32_t N,
                                     int32_t value_dtype, int32_t rows_per_window, ra_stream_t stream,
                                     ra_tile_plan** out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: out is NULL");
    *out = nullptr;
    if (kind < RA_TILE_TC_DIRECT || kind > RA_TILE_SEGMENT_HYBRID)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: unknown kind");
    if (value_dtype != RA_DTYPE_F16 && value_dtype != RA_DTYPE_BF16)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: value_dtype must be F16 or BF16");
    if (M < 0 || K < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: negative dimension");
    if (M > 0 && !d_rowptr) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: rowptr is NULL");
    const auto t0 = std::chrono::steady_clock::now();
    auto p = new (std::nothrow) ra_tile_plan();
    if (!p) return ra::fail(RA_ERR_OUT_OF_MEMORY, "tile: plan allocation");
    if (rows_per_window != 0 && rows_per_window != 8 && rows_per_window != 16 && rows_per_window != 32) {
        delete p;
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: rows_per_window must be 0 (auto), 8, 16 or 32");
    }
    const ra_status s = gpu_build(p, kind, d_rowptr, d_colind, d_vals, M, K, N, value_dtype, rows_per_window,
                                  reinterpret_cast<hipStream_t>(stream));
    if (s != RA_OK) {
        delete p;
        return s;
    }
    p->info.build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    *out = p;
    return RA_OK;
}

ra_status ra_tile_plan_export(const ra_tile_plan* p, const char* name, void* dst, int64_t* count) {
    if (!p || !name || !count) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile export: NULL argument");
    size_t elem = 4;
    int64_t n = 0;
    const ra::DeviceBuffer* b = plan_array(p, name, elem, n);
    if (!b) return ra::fail(RA_ERR_INVALID_ARGUMENT, std::string("tile export: unknown array '") + name + "'");
    *count = n;
    if (dst && n > 0) RA_HIP_TRY(hipMemcpy(dst, b->get(), n * elem, hipMemcpyDeviceToHost));
    return RA_OK;
}

}  // extern "C"
