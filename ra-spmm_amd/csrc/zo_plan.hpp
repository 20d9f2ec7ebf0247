// zo_plan.hpp — ZERO_OVERHEAD_CSR plan shared by the host binning
// (csr_kernels.hip) and the device binning (zo_build_gpu.hip).
//
// Bins of csr/ra_zero_overhead.cu:331-358: empty, tiny (<= 4 nnz), short
// (<= 16), medium (<= 64), long (> 64) cut into 256-nnz chunks; bit 31 of a
// chunk's row marks a sole chunk (rows of 65..256 nnz, written directly).
#pragma once

#include <algorithm>
#include <cstdint>

#include "../../include/ra_spmm.h"
#include "ra_internal.hpp"

namespace ra {
constexpr int kTiny = 4, kShort = 16, kMedium = 64, kChunk = 256;
constexpr uint32_t kSoleFlag = 0x80000000u;
}  // namespace ra

// short_rows = empty rows, then tiny, short, medium rows, each ascending.
// chunk_rows/chunk_starts/chunk_slot: one entry per chunk, rows ascending and
// a row's chunks consecutive; split chunks own consecutive partial slots
// (chunk_slot, -1 for sole chunks), merged per split row over
// [split_off[i], split_off[i+1]).
struct ra_zo_plan {
    ra_zo_info info{};
    int device = 0;
    // The six lists live in one allocation (one hipMalloc per build, one
    // hipFree per plan): short_rows | chunk_rows | chunk_starts | chunk_slot |
    // split_rows | split_off, each 256-byte aligned.
    ra::DeviceBuffer lists;
    int32_t *short_rows = nullptr, *chunk_rows = nullptr, *chunk_starts = nullptr, *chunk_slot = nullptr,
            *split_rows = nullptr, *split_off = nullptr;
    ra::DeviceBuffer partials;  // grown per N, reused across runs
    int64_t num_short_total = 0; // empty + tiny + short + medium

    ra_status carve(int64_t n_short, int64_t n_chunks, int64_t n_split) {
        const int64_t counts[6] = {n_short, n_chunks, n_chunks, n_chunks, n_split, n_split + 1};
        auto round = [](int64_t n) { return (static_cast<size_t>(std::max<int64_t>(n, 1)) * 4 + 255) & ~size_t(255); };
        size_t total = 0;
        for (int64_t c : counts) total += round(c);
        RA_TRY(lists.allocate(total));
        int32_t** dst[6] = {&short_rows, &chunk_rows, &chunk_starts, &chunk_slot, &split_rows, &split_off};
        size_t off = 0;
        for (int i = 0; i < 6; ++i) {
            *dst[i] = reinterpret_cast<int32_t*>(lists.get<char>() + off);
            off += round(counts[i]);
        }
        return RA_OK;
    }
};

namespace ra {
// ZERO_OVERHEAD_CSR run (both launches) with the split chunks' partial slots in
// `partials` ([num_split_chunks][N] fp32, 16-byte aligned) instead of the
// plan's own buffer (csr_kernels.hip).
ra_status zo_run_with_partials(ra_zo_plan* plan, const int32_t* d_rowptr, const int32_t* d_colind,
                               const float* d_vals, const float* d_B, float* d_C, int32_t N, float* partials,
                               hipStream_t st);
}  // namespace ra
