// zo_noalloc.hip — the ZERO_OVERHEAD_CSR run that allocates nothing.
//
// ra_zo_plan_run_noalloc keeps the split rows' partial slots in a fixed
// device array instead of a plan-owned allocation, for callers that cannot
// allocate device memory.  Every GPU the library runs on holds its own copy of
// the array for the life of the process, once this file's code object is
// loaded (on the first no-alloc call: it lives in its own translation unit so
// that no other entry point pays the 64 MiB at load time).  Calls on one GPU
// share the array; each call writes every slot it reads, so nothing needs
// clearing, and calls that overlap on one GPU race.  Host code never passes
// the array's name to a kernel: it takes the device address from
// hipGetSymbolAddress, once per device, and uses that.
#include <cstdint>
#include <mutex>

#include "ra_internal.hpp"
#include "zo_plan.hpp"

namespace {

constexpr uint64_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mutex;
void* g_scratch_ptr[64] = {};

ra_status noalloc_scratch(void** out) {
    int dev = 0;
    RA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return ra::fail(RA_ERR_UNSUPPORTED, "noalloc scratch: device id >= 64");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return ra::fail(RA_ERR_HIP, "noalloc scratch: hipGetSymbolAddress failed");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return RA_OK;
}

}  // namespace

extern "C" {

ra_status ra_zo_plan_run_noalloc(ra_zo_plan* plan, const int32_t* d_rowptr,
                                 const int32_t* d_colind, const float* d_vals, const float* d_B,
                                 float* d_C, int32_t N, ra_stream_t stream) {
    if (!plan) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo noalloc: plan is NULL");
    if (N < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo noalloc: N < 0");
    const uint64_t need = (uint64_t)plan->info.num_split_chunks * (uint64_t)N * sizeof(float);
    if (need > kNoAllocScratchBytes)
        return ra::fail(RA_ERR_UNSUPPORTED,
                        "zo noalloc: the split rows need more partial-slot memory than the "
                        "fixed 64 MiB scratch (num_split_chunks * N * 4 bytes)");
    float* slots = nullptr;
    if (need > 0) RA_TRY(noalloc_scratch(reinterpret_cast<void**>(&slots)));
    return ra::zo_run_with_partials(plan, d_rowptr, d_colind, d_vals, d_B, d_C, N, slots,
                                    reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
