// common.cpp — error state, names and the host parallel_for of the C ABI.
#include <algorithm>
#include <atomic>
#include <thread>

#include "ra_internal.hpp"

namespace ra {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

void parallel_for(int64_t n, int64_t grain, const std::function<void(int64_t, int64_t)>& f) {
    if (n <= 0) return;
    grain = std::max<int64_t>(1, grain);
    const int64_t chunks = (n + grain - 1) / grain;
    unsigned hw = std::thread::hardware_concurrency();
    if (hw == 0) hw = 1;
    const int64_t nthreads = std::min<int64_t>(std::min<int64_t>(hw, 64), chunks);
    if (nthreads <= 1) {
        f(0, n);
        return;
    }
    std::atomic<int64_t> next{0};
    auto worker = [&]() {
        for (;;) {
            const int64_t c = next.fetch_add(1);
            if (c >= chunks) break;
            const int64_t b = c * grain;
            f(b, std::min(n, b + grain));
        }
    };
    std::vector<std::thread> pool;
    pool.reserve(nthreads - 1);
    for (int64_t t = 1; t < nthreads; ++t) pool.emplace_back(worker);
    worker();
    for (auto& t : pool) t.join();
}

}  // namespace ra

extern "C" {

int ra_abi_version(void) { return RA_SPMM_ABI_VERSION; }

const char* ra_last_error(void) { return ra::g_last_error.c_str(); }

const char* ra_status_string(ra_status s) {
    switch (s) {
        case RA_OK: return "RA_OK";
        case RA_ERR_INVALID_ARGUMENT: return "RA_ERR_INVALID_ARGUMENT";
        case RA_ERR_HIP: return "RA_ERR_HIP";
        case RA_ERR_OUT_OF_MEMORY: return "RA_ERR_OUT_OF_MEMORY";
        case RA_ERR_UNSUPPORTED: return "RA_ERR_UNSUPPORTED";
        case RA_ERR_INACTIVE_PLAN: return "RA_ERR_INACTIVE_PLAN";
        case RA_ERR_INTERNAL: return "RA_ERR_INTERNAL";
    }
    return "RA_ERR_UNKNOWN";
}

// Path names keep the reference spelling (ra_common.h:116-135) because the
// router dict, the Python mirror and the harness labels all key on them.
const char* ra_path_name(int32_t p) {
    static const char* const kNames[RA_PATH_COUNT] = {
        "CSR_DIRECT",   "CSR_ADAPTIVE",      "STAGED_REUSE",   "TC_SPARSE",
        "ROW_SPLIT_CUDA", "TC_REORDERED",    "HYBRID_TC_CUDA", "CUSPARSE",
        "RODE_ENHANCED", "VECTORIZED_COARSE", "LOCALITY_TILED", "TC_DIRECT",
        "COMMUNITY_TC", "ZERO_OVERHEAD_CSR", "SEGMENT_HYBRID"};
    if (p < 0 || p >= RA_PATH_COUNT) return "UNKNOWN";
    return kNames[p];
}

// Rejection names keep the reference spelling (ra_common.h:161-178).
const char* ra_reject_name(int32_t c) {
    static const char* const kNames[] = {
        "CHOSEN",         "NOT_FEASIBLE",     "LOW_FILL",          "LOW_COVERAGE",
        "HIGH_SKEW",      "SMALL_N",          "INSUFFICIENT_NNZ",  "LOW_OCCUPANCY",
        "LOW_DEGREE_SKEW", "NOT_STRONG_ENOUGH", "MARGIN_TOO_SMALL", "NOT_IN_PORTFOLIO",
        "UNKNOWN"};
    if (c < 0 || c > RA_REJECT_UNKNOWN) return "UNKNOWN";
    return kNames[c];
}

}  // extern "C"
