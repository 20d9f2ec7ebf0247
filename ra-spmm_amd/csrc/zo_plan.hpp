// zo_plan.hpp — ZERO_OVERHEAD_CSR plan shared by the host binning
// (csr_kernels.hip) and the device binning (zo_build_gpu.hip).
//
// Bins of csr/ra_zero_overhead.cu:331-358: empty, tiny (<= 4 nnz), short
// (<= 16), medium (<= 64), long (> 64) cut into 256-nnz chunks; bit 31 of a
// chunk's row marks a sole chunk (rows of 65..256 nnz, written directly).
#pragma once

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
    ra::DeviceBuffer chunk_rows, chunk_starts, chunk_slot, short_rows, split_rows, split_off;
    ra::DeviceBuffer partials;  // grown per N, reused across runs
    int64_t num_short_total = 0; // empty + tiny + short + medium
};
