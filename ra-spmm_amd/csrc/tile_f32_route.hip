// tile_f32_route.hip — the FP32 route of the tile plans (the `_tf32` entry
// points) as a CSR SpMM over the plan's stored values.
//
// The reference's TF32 route runs its tile kernel with TF32 MMA
// (tc/ra_tc_direct.cu:189-261); gfx950 has no xf32 MFMA, so this build's FP32
// route computes exact fp32 fma of the stored (fp16/bf16-rounded, scaled-back)
// values and fp32 B.  Done on the 8x8 / 32-row blocks, 85-95% of those fmas
// multiply padding zeros and every block re-reads its A values; the same
// products in CSR form run on the CSR kernels at the gather rate.  So on the
// first FP32-route call a plan derives, on the device:
//   1. per vector, the number of nonzero stored values (count pass, then scan)
//   2. one key (row << cb | column, cb = bits of K - 1) and exact fp32 value
//      per stored nonzero
//   3. a radix sort of (key, value): rows ascending, columns ascending within
//      a row (a plan holds each (row, column) once: duplicates were summed)
//   4. rowptr from the last index of each row and a max-scan (no atomics)
// and keeps (rowptr, colind, vals).  Every later call runs CSR_DIRECT on them:
// one fp32 fma chain per output element in ascending column order, the same
// chain the tile kernels computed, bit for bit.  A plan with column partitions
// keeps them: one CSR per column range, launched in order, each continuing
// the chains the previous one left in C (the B rows in use stay K / P).  Rows of skewed length
// (degree CV >= 1.5, the router's own ZERO_OVERHEAD_CSR threshold) run on a
// ZERO_OVERHEAD_CSR plan instead, which keeps rows of <= 256 nonzeros
// bit-exact and sums longer rows in 256-nonzero chunks.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>
#include <cmath>

#include "ra_internal.hpp"
#include "tile_format.hpp"

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 20)));
}

#define RA_GRID_STRIDE(i, n) \
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

__global__ void f32_fill_i32(int32_t* p, int64_t n, int32_t v) { RA_GRID_STRIDE(i, n) p[i] = v; }

__device__ __forceinline__ float stored_value(uint16_t h, bool bf16, float unscale) {
    if (bf16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, h)) * unscale;  // exact: power of two
}

// Offset of stored value (slot, vector kk) in a block: 8-row blocks are
// [slot][vector]; tall blocks [slot/16][vector/8][slot%16][vector%8].
__device__ __forceinline__ int64_t value_at(int64_t blk, int slot, int kk, int H, int vb) {
    return vb == 8 ? blk * 64 + slot * 8 + kk
                   : blk * ((int64_t)H * 32) + ((((slot >> 4) * 4 + (kk >> 3)) * 16 + (slot & 15)) * 8 + (kk & 7));
}

// Cell (window, or partition * W + window) of block b: last c with
// block_offsets[c] <= b.
__device__ __forceinline__ int64_t cell_of(const int32_t* __restrict__ boff, int64_t ncells, int64_t b) {
    int64_t lo = 0, hi = ncells - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (boff[mid] <= b) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Pass 1: nonzero stored values of every vector.  Pass 2 (emit): their keys
// and values at the vector's offset.
// With column partitions kept (parts > 1) the key's row is part * M + row, so
// the sorted CSR holds partition 0's rows, then partition 1's, ...
template <bool EMIT>
__global__ void vector_entries(const int32_t* __restrict__ boff, int64_t ncells, int64_t W,
                               const int32_t* __restrict__ atox, const uint16_t* __restrict__ vals,
                               const int32_t* __restrict__ win_rows, int64_t nvec, int H, int vb, int bf16,
                               float unscale, int parts, int64_t M, int cb, int32_t* __restrict__ count,
                               const int32_t* __restrict__ offset, uint64_t* __restrict__ keys,
                               float* __restrict__ out) {
    RA_GRID_STRIDE(v, nvec) {
        const int32_t col = atox[v];
        int n = 0;
        if (col >= 0) {
            const int64_t b = v / vb;
            const int kk = static_cast<int>(v - b * vb);
            int64_t o = EMIT ? offset[v] : 0;
            int64_t w = 0, part = 0;
            if (EMIT) {
                const int64_t cell = cell_of(boff, ncells, b);
                w = cell % W;
                part = parts > 1 ? cell / W : 0;
            }
            for (int slot = 0; slot < H; ++slot) {
                const uint16_t h = vals[value_at(b, slot, kk, H, vb)];
                if ((h & 0x7FFFu) == 0) continue;  // +0 / -0: no product
                if (EMIT) {
                    const int64_t row = part * M + win_rows[w * H + slot];
                    keys[o] = (static_cast<uint64_t>(row) << cb) | static_cast<uint32_t>(col);
                    out[o] = stored_value(h, bf16 != 0, unscale);
                    ++o;
                } else {
                    ++n;
                }
            }
        }
        if (!EMIT) count[v] = n;
    }
}

// last[row] = 1 + index of the row's last entry (rows without entries stay 0;
// the max-scan then carries the previous row's end).
__global__ void row_ends(const uint64_t* __restrict__ keys, int64_t n, int cb, int32_t* __restrict__ last,
                         int32_t* __restrict__ colind) {
    RA_GRID_STRIDE(i, n) {
        const uint64_t k = keys[i];
        const int64_t row = static_cast<int64_t>(k >> cb);
        colind[i] = static_cast<int32_t>(k & ((uint64_t(1) << cb) - 1));
        if (i == n - 1 || (keys[i + 1] >> cb) != static_cast<uint64_t>(row)) last[row] = static_cast<int32_t>(i + 1);
    }
}

}  // namespace

namespace ra {

// Degree CV at or above which the FP32 route runs ZERO_OVERHEAD_CSR (the
// MI355X router table's zo_min_cv).
constexpr float kF32RouteZoCv = 1.5f;

ra_status tile_f32_prepare(ra_tile_plan* p, hipStream_t st) {
    if (p->f32_ready) return RA_OK;
    const ra_tile_info& I = p->info;
    const int M = I.M;
    const int H = I.rows_per_window > 0 ? I.rows_per_window : kTileWindow;
    const int vb = H == kTileWindow ? kTileVec : 32;
    const int64_t W = I.num_windows;
    const int64_t ncells = W * std::max(I.col_parts, 1);
    const int64_t nvec = (int64_t)I.num_blocks * vb;
    const float unscale = std::ldexp(1.0f, -I.value_scale_log2);
    const int bf16 = I.value_dtype == RA_DTYPE_BF16 ? 1 : 0;
    // Column partitions of the plan are kept (one CSR per column range, run in
    // order) when the (part * M + row, column) key fits 64 bits.
    int cb = 1;  // columns are < K <= 2^cb
    while ((int64_t(1) << cb) < I.K) ++cb;
    int parts = std::max(I.col_parts, 1);
    int rbits = 1;
    while ((int64_t(1) << rbits) < (int64_t)parts * M) ++rbits;
    if (cb + rbits > 64 || (int64_t)parts * M >= INT32_MAX) {
        parts = 1;
        rbits = 1;
        while ((int64_t(1) << rbits) < M) ++rbits;
    }
    const int64_t R = (int64_t)parts * M;  // rows of the derived CSR

    // Per-vector counts and their exclusive scan (nvec + 1 entries: the last is the total).
    DeviceBuffer cnt, off;
    RA_TRY(cnt.allocate((nvec + 1) * sizeof(int32_t)));
    RA_TRY(off.allocate((nvec + 1) * sizeof(int32_t)));
    f32_fill_i32<<<1, kThreads, 0, st>>>(cnt.get<int32_t>() + nvec, 1, 0);
    if (nvec > 0)
        vector_entries<false><<<grid_for(nvec), kThreads, 0, st>>>(
            p->block_offsets.get<int32_t>(), ncells, W, p->atox.get<int32_t>(), p->vals.get<uint16_t>(),
            p->win_rows.get<int32_t>(), nvec, H, vb, bf16, unscale, parts, M, cb, cnt.get<int32_t>(), nullptr,
            nullptr, nullptr);
    RA_LAUNCH_CHECK("vector_entries count");
    size_t tb = 0;
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, tb, cnt.get<int32_t>(), off.get<int32_t>(),
                                                static_cast<int>(nvec + 1), st));
    DeviceBuffer tmp;
    RA_TRY(tmp.allocate(std::max<size_t>(tb, 1)));
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(tmp.get(), tb, cnt.get<int32_t>(), off.get<int32_t>(),
                                                static_cast<int>(nvec + 1), st));
    int32_t total = 0;
    RA_HIP_TRY(hipMemcpyAsync(&total, off.get<int32_t>() + nvec, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    RA_HIP_TRY(hipStreamSynchronize(st));
    const int64_t n = total;

    // Keys and values, sorted by (row, column).
    DeviceBuffer keys, keys2, v1;
    RA_TRY(keys.allocate(std::max<int64_t>(n, 1) * sizeof(uint64_t)));
    RA_TRY(keys2.allocate(std::max<int64_t>(n, 1) * sizeof(uint64_t)));
    RA_TRY(v1.allocate(std::max<int64_t>(n, 1) * sizeof(float)));
    RA_TRY(p->f32_vals.allocate(std::max<int64_t>(n, 1) * sizeof(float)));
    RA_TRY(p->f32_colind.allocate(std::max<int64_t>(n, 1) * sizeof(int32_t)));
    RA_TRY(p->f32_rowptr.allocate((R + 1) * sizeof(int32_t)));
    int32_t* rowptr = p->f32_rowptr.get<int32_t>();
    f32_fill_i32<<<grid_for(R + 1), kThreads, 0, st>>>(rowptr, R + 1, 0);
    if (n > 0) {
        vector_entries<true><<<grid_for(nvec), kThreads, 0, st>>>(
            p->block_offsets.get<int32_t>(), ncells, W, p->atox.get<int32_t>(), p->vals.get<uint16_t>(),
            p->win_rows.get<int32_t>(), nvec, H, vb, bf16, unscale, parts, M, cb, nullptr, off.get<int32_t>(),
            keys.get<uint64_t>(), v1.get<float>());
        RA_LAUNCH_CHECK("vector_entries emit");
        size_t sb = 0;
        RA_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sb, keys.get<uint64_t>(), keys2.get<uint64_t>(),
                                                      v1.get<float>(), p->f32_vals.get<float>(),
                                                      static_cast<int>(n), 0, cb + rbits, st));
        RA_TRY(tmp.ensure(std::max<size_t>(sb, 1)));
        RA_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(tmp.get(), sb, keys.get<uint64_t>(), keys2.get<uint64_t>(),
                                                      v1.get<float>(), p->f32_vals.get<float>(),
                                                      static_cast<int>(n), 0, cb + rbits, st));
        // last[row] = end of the row's entries; a max-scan into rowptr[1..M]
        // fills the rows without entries.
        DeviceBuffer last;
        RA_TRY(last.allocate(static_cast<size_t>(R) * sizeof(int32_t)));
        f32_fill_i32<<<grid_for(R), kThreads, 0, st>>>(last.get<int32_t>(), R, 0);
        row_ends<<<grid_for(n), kThreads, 0, st>>>(keys2.get<uint64_t>(), n, cb, last.get<int32_t>(),
                                                   p->f32_colind.get<int32_t>());
        RA_LAUNCH_CHECK("row_ends");
        size_t ms = 0;
        RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(nullptr, ms, last.get<int32_t>(), rowptr + 1, hipcub::Max(),
                                                     static_cast<int>(R), st));
        RA_TRY(tmp.ensure(std::max<size_t>(ms, 1)));
        RA_HIP_TRY(hipcub::DeviceScan::InclusiveScan(tmp.get(), ms, last.get<int32_t>(), rowptr + 1, hipcub::Max(),
                                                     static_cast<int>(R), st));
        RA_HIP_TRY(hipStreamSynchronize(st));  // before `last`, `keys*`, `v1` and `tmp` are freed
    }
    p->f32_nnz = n;
    p->f32_parts = parts;

    // Skewed rows (one column range): a ZERO_OVERHEAD_CSR plan over the derived rowptr.
    if (parts == 1) {
        ra_features f{};
        RA_TRY(ra_features_device(rowptr, M, I.K, 16, reinterpret_cast<ra_stream_t>(st), &f));
        if (f.degree_cv >= kF32RouteZoCv)
            RA_TRY(ra_zo_plan_create_device(rowptr, M, I.K, reinterpret_cast<ra_stream_t>(st), &p->f32_zo));
    }
    RA_HIP_TRY(hipStreamSynchronize(st));
    p->f32_ready = true;
    return RA_OK;
}

ra_status tile_f32_run(ra_tile_plan* p, const float* B, float* C, int32_t N, hipStream_t st) {
    RA_TRY(tile_f32_prepare(p, st));
    const ra_stream_t s = reinterpret_cast<ra_stream_t>(st);
    if (p->f32_zo)
        return ra_zo_plan_run(p->f32_zo, p->f32_rowptr.get<int32_t>(), p->f32_colind.get<int32_t>(),
                              p->f32_vals.get<float>(), B, C, N, s);
    // Column ranges in ascending order; each continues the fma chains the
    // previous one stored in C, so the result is the single chain per element.
    const int64_t M = p->info.M;
    for (int q = 0; q < p->f32_parts; ++q)
        RA_TRY(csr_direct_launch(p->f32_rowptr.get<int32_t>() + q * M, p->f32_colind.get<int32_t>(),
                                 p->f32_vals.get<float>(), B, C, p->info.M, p->info.K, N, p->f32_nnz, q > 0, st));
    return RA_OK;
}

}  // namespace ra
