// zo_build_gpu.hip — device binning of the ZERO_OVERHEAD_CSR plan (cold path).
//
// Same lists as the host binning (ra_zo_bins_host + ra_zo_plan_create in
// csr_kernels.hip), produced from a device rowptr in three launches and one
// scan: classify every row (bin, chunks, split), exclusive-scan the per-row
// counters, scatter each row to its list positions.  Reference algorithm:
// make_ra_zero_overhead_plan, csr/ra_zero_overhead.cu:312-387 (a host loop).
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <string>

#include "ra_internal.hpp"
#include "zo_plan.hpp"

namespace {

constexpr int kThreads = 256;

// Per-row counters, scanned together: rows per bin (empty, tiny, short,
// medium), chunks, split rows, split chunks, sole chunks.
struct alignas(16) ZoCounts {
    int32_t c[8];
};

struct ZoCountsSum {
    __host__ __device__ ZoCounts operator()(const ZoCounts& a, const ZoCounts& b) const {
        ZoCounts r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.c[i] = a.c[i] + b.c[i];
        return r;
    }
};

enum { kEmpty = 0, kTinyBin = 1, kShortBin = 2, kMediumBin = 3, kChunks = 4, kSplitRows = 5,
       kSplitChunks = 6, kSoleChunks = 7 };

// counts[i] for rows i < M, counts[M] = 0 so the exclusive scan's last entry
// is the total.  flags[0]: non-monotone rows.  block_max[b]: longest row of
// workgroup b, reduced by block_max_reduce: atomics on one address, one per
// wave, serialised to ~185 us on 1e6 rows on MI355X (none: ~24 us).
__global__ void zo_classify(const int32_t* __restrict__ rowptr, int M, ZoCounts* __restrict__ counts,
                            unsigned* __restrict__ flags, unsigned* __restrict__ block_max) {
    __shared__ unsigned part[kThreads / 64];
    unsigned longest = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= M;
         i += (int64_t)gridDim.x * blockDim.x) {
        ZoCounts v;
#pragma unroll
        for (int k = 0; k < 8; ++k) v.c[k] = 0;
        if (i < M) {
            const int64_t d = (int64_t)rowptr[i + 1] - rowptr[i];
            if (d < 0) atomicAdd(&flags[0], 1u);
            else if (d == 0) v.c[kEmpty] = 1;
            else if (d <= ra::kTiny) v.c[kTinyBin] = 1;
            else if (d <= ra::kShort) v.c[kShortBin] = 1;
            else if (d <= ra::kMedium) v.c[kMediumBin] = 1;
            else {
                const int nch = static_cast<int>((d + ra::kChunk - 1) / ra::kChunk);
                v.c[kChunks] = nch;
                if (nch == 1) v.c[kSoleChunks] = 1;
                else {
                    v.c[kSplitRows] = 1;
                    v.c[kSplitChunks] = nch;
                }
                longest = max(longest, static_cast<unsigned>(d));
            }
        }
        counts[i] = v;
    }
    for (int off = 32; off > 0; off >>= 1) longest = max(longest, __shfl_xor(longest, off, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = longest;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) longest = max(longest, part[w]);
        block_max[blockIdx.x] = longest;
    }
}

// out = max over block_max[0, n): one workgroup.
__global__ void block_max_reduce(const unsigned* __restrict__ block_max, int n, unsigned* __restrict__ out) {
    __shared__ unsigned part[kThreads / 64];
    unsigned m = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = max(m, block_max[i]);
    for (int off = 32; off > 0; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) m = max(m, part[w]);
        *out = m;
    }
}

__global__ void zo_scatter(const int32_t* __restrict__ rowptr, int M, const ZoCounts* __restrict__ pre,
                           int4 bin_base, int32_t* __restrict__ short_rows, int32_t* __restrict__ chunk_rows,
                           int32_t* __restrict__ chunk_starts, int32_t* __restrict__ chunk_slot,
                           int32_t* __restrict__ split_rows, int32_t* __restrict__ split_off) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < M;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int32_t start = rowptr[i];
        const int64_t d = (int64_t)rowptr[i + 1] - start;
        const ZoCounts& o = pre[i];
        if (d == 0) short_rows[bin_base.x + o.c[kEmpty]] = static_cast<int32_t>(i);
        else if (d <= ra::kTiny) short_rows[bin_base.y + o.c[kTinyBin]] = static_cast<int32_t>(i);
        else if (d <= ra::kShort) short_rows[bin_base.z + o.c[kShortBin]] = static_cast<int32_t>(i);
        else if (d <= ra::kMedium) short_rows[bin_base.w + o.c[kMediumBin]] = static_cast<int32_t>(i);
        else {
            const int nch = static_cast<int>((d + ra::kChunk - 1) / ra::kChunk);
            const bool sole = nch == 1;
            const int32_t tag = sole ? static_cast<int32_t>(static_cast<uint32_t>(i) | ra::kSoleFlag)
                                     : static_cast<int32_t>(i);
            for (int k = 0; k < nch; ++k) {
                const int c = o.c[kChunks] + k;
                chunk_rows[c] = tag;
                chunk_starts[c] = start + k * ra::kChunk;
                chunk_slot[c] = sole ? -1 : o.c[kSplitChunks] + k;
            }
            if (!sole) {
                split_rows[o.c[kSplitRows]] = static_cast<int32_t>(i);
                split_off[o.c[kSplitRows] + 1] = o.c[kSplitChunks] + nch;
            }
        }
        if (i == 0) split_off[0] = 0;
    }
}

__global__ void zero_flags(unsigned* flags) {
    if (threadIdx.x < 2) flags[threadIdx.x] = 0u;
}

constexpr size_t kCachedTmpBytes = size_t(256) << 20;
constexpr int kMaxDevices = 64;
std::mutex g_tmp_mutex;
ra::DeviceBuffer* g_tmp[kMaxDevices] = {};

unsigned grid_for(int64_t n) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 16)));
}

ra_status gpu_bin(ra_zo_plan* p, const int32_t* rowptr, int32_t M, int32_t K, hipStream_t st) {
    ra_zo_info& z = p->info;
    z = ra_zo_info{};
    z.M = M;
    z.K = K;
    (void)hipGetDevice(&p->device);
    if (M == 0) return RA_OK;
    size_t scan_bytes = 0;
    ZoCounts* cnull = nullptr;
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveScan(nullptr, scan_bytes, cnull, cnull, ZoCountsSum(), ZoCounts{},
                                                 M + 1, st));
    const size_t counts_bytes = ((size_t)(M + 1) * sizeof(ZoCounts) + 255) & ~size_t(255);
    const unsigned cgrid = grid_for(M + 1);
    const size_t tmp_bytes =
        2 * counts_bytes + ((scan_bytes + 255) & ~size_t(255)) + 256 + (size_t)cgrid * sizeof(unsigned);
    // The counters come from a per-device buffer kept for the process (up to
    // kCachedTmpBytes; a hipMalloc + hipFree pair costs a cold build
    // ~0.3 ms); larger builds allocate their own.  Builds on one device are
    // serialised by the buffer's lock.
    ra::DeviceBuffer own;
    std::unique_lock<std::mutex> lock;
    ra::DeviceBuffer* tmpp = &own;
    if (tmp_bytes <= kCachedTmpBytes && p->device >= 0 && p->device < kMaxDevices) {
        lock = std::unique_lock<std::mutex>(g_tmp_mutex);
        if (!g_tmp[p->device]) g_tmp[p->device] = new ra::DeviceBuffer();  // kept until exit
        tmpp = g_tmp[p->device];
        RA_TRY(tmpp->ensure(tmp_bytes));
    } else {
        RA_TRY(own.allocate(tmp_bytes));
    }
    ra::DeviceBuffer& tmp = *tmpp;
    ZoCounts* counts = tmp.get<ZoCounts>();
    ZoCounts* pre = reinterpret_cast<ZoCounts*>(tmp.get<char>() + counts_bytes);
    void* scan_tmp = tmp.get<char>() + 2 * counts_bytes;
    unsigned* flags = reinterpret_cast<unsigned*>(tmp.get<char>() + 2 * counts_bytes +
                                                  ((scan_bytes + 255) & ~size_t(255)));
    unsigned* block_max = flags + 64;  // after the 256-byte flags slot
    zero_flags<<<1, 64, 0, st>>>(flags);
    zo_classify<<<cgrid, kThreads, 0, st>>>(rowptr, M, counts, flags, block_max);
    block_max_reduce<<<1, kThreads, 0, st>>>(block_max, static_cast<int>(cgrid), flags + 1);
    RA_LAUNCH_CHECK("zo_classify");
    RA_HIP_TRY(hipcub::DeviceScan::ExclusiveScan(scan_tmp, scan_bytes, counts, pre, ZoCountsSum(), ZoCounts{},
                                                 M + 1, st));
    ZoCounts tot;
    unsigned hflags[2];
    RA_HIP_TRY(hipMemcpyAsync(&tot, pre + M, sizeof(tot), hipMemcpyDeviceToHost, st));
    RA_HIP_TRY(hipMemcpyAsync(hflags, flags, sizeof(hflags), hipMemcpyDeviceToHost, st));
    RA_HIP_TRY(hipStreamSynchronize(st));
    if (hflags[0]) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: rowptr not monotone");

    z.num_empty = tot.c[kEmpty];
    z.num_tiny = tot.c[kTinyBin];
    z.num_short = tot.c[kShortBin];
    z.num_medium = tot.c[kMediumBin];
    z.num_small = z.num_tiny + z.num_short + z.num_medium;
    z.num_chunks = tot.c[kChunks];
    z.num_sole_chunks = tot.c[kSoleChunks];
    z.num_split_rows = tot.c[kSplitRows];
    z.num_split_chunks = tot.c[kSplitChunks];
    z.num_long = z.num_sole_chunks + z.num_split_rows;
    z.max_long_chunks = static_cast<int32_t>((static_cast<int64_t>(hflags[1]) + ra::kChunk - 1) / ra::kChunk);
    z.plan_bytes = (int64_t)sizeof(int32_t) *
                   ((int64_t)z.num_small + z.num_empty + 3LL * z.num_chunks + 2LL * z.num_split_rows + 1);
    p->num_short_total = (int64_t)z.num_empty + z.num_small;

    RA_TRY(p->carve(p->num_short_total, z.num_chunks, z.num_split_rows));
    const int4 base{0, z.num_empty, z.num_empty + z.num_tiny, z.num_empty + z.num_tiny + z.num_short};
    zo_scatter<<<grid_for(M), kThreads, 0, st>>>(rowptr, M, pre, base, p->short_rows, p->chunk_rows,
                                                 p->chunk_starts, p->chunk_slot, p->split_rows, p->split_off);
    RA_LAUNCH_CHECK("zo_scatter");
    RA_HIP_TRY(hipStreamSynchronize(st));
    return RA_OK;
}

}  // namespace

extern "C" {

ra_status ra_zo_plan_create_device(const int32_t* d_rowptr, int32_t M, int32_t K, ra_stream_t stream,
                                   ra_zo_plan** out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: out is NULL");
    *out = nullptr;
    if (M < 0 || (M > 0 && !d_rowptr)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: bad rowptr");
    auto p = new (std::nothrow) ra_zo_plan();
    if (!p) return ra::fail(RA_ERR_OUT_OF_MEMORY, "zo: plan allocation");
    const ra_status s = gpu_bin(p, d_rowptr, M, K, reinterpret_cast<hipStream_t>(stream));
    if (s != RA_OK) {
        delete p;
        return s;
    }
    *out = p;
    return RA_OK;
}

ra_status ra_zo_plan_export(const ra_zo_plan* p, const char* name, int32_t* dst, int64_t* count) {
    if (!p || !name || !count) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo export: NULL argument");
    const std::string n(name);
    const ra_zo_info& z = p->info;
    const int32_t* b = nullptr;
    int64_t c = 0;
    if (n == "short_rows") { b = p->short_rows; c = p->num_short_total; }
    else if (n == "chunk_rows") { b = p->chunk_rows; c = z.num_chunks; }
    else if (n == "chunk_starts") { b = p->chunk_starts; c = z.num_chunks; }
    else if (n == "chunk_slot") { b = p->chunk_slot; c = z.num_chunks; }
    else if (n == "split_rows") { b = p->split_rows; c = z.num_split_rows; }
    else if (n == "split_off") { b = p->split_off; c = z.M > 0 ? z.num_split_rows + 1 : 0; }
    else return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo export: unknown array '" + n + "'");
    *count = c;
    if (dst && c > 0) RA_HIP_TRY(hipMemcpy(dst, b, c * sizeof(int32_t), hipMemcpyDeviceToHost));
    return RA_OK;
}

}  // extern "C"
