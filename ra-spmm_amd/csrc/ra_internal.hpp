// ra_internal.hpp — shared plumbing of the C ABI (error state, HIP checks,
// device-buffer RAII).  Not part of the public interface (include/ra_spmm.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ra_spmm.h"

namespace ra {

// Thread-local message behind ra_last_error().
void set_error(const std::string& msg);
void clear_error();

inline ra_status fail(ra_status s, const std::string& msg) {
    set_error(msg);
    return s;
}

inline ra_status hip_fail(hipError_t e, const char* what) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? RA_ERR_OUT_OF_MEMORY : RA_ERR_HIP;
}

#define RA_HIP_TRY(expr)                                        \
    do {                                                        \
        hipError_t _e = (expr);                                 \
        if (_e != hipSuccess) return ::ra::hip_fail(_e, #expr); \
    } while (0)

#define RA_TRY(expr)                              \
    do {                                          \
        ra_status _s = (expr);                    \
        if (_s != RA_OK) return _s;               \
    } while (0)

// Launch check: a bad launch configuration surfaces here, not at the next sync.
#define RA_LAUNCH_CHECK(what)                                        \
    do {                                                             \
        hipError_t _e = hipGetLastError();                           \
        if (_e != hipSuccess) return ::ra::hip_fail(_e, what);       \
    } while (0)

// Owning device allocation (hipMalloc / hipFree).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    ~DeviceBuffer() { reset(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
        o.ptr_ = nullptr;
        o.bytes_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            std::swap(ptr_, o.ptr_);
            std::swap(bytes_, o.bytes_);
        }
        return *this;
    }

    ra_status allocate(size_t bytes) {
        reset();
        if (bytes == 0) return RA_OK;
        // RA_MAX_ALLOC_BYTES caps one allocation (read per call): a larger one
        // fails as out of memory, so the failure paths can be exercised on a
        // GPU with plenty of memory.
        if (const char* cap = std::getenv("RA_MAX_ALLOC_BYTES")) {
            if (bytes > std::strtoull(cap, nullptr, 10))
                return fail(RA_ERR_OUT_OF_MEMORY, "hipMalloc: " + std::to_string(bytes) +
                                                      " bytes exceed RA_MAX_ALLOC_BYTES");
        }
        hipError_t e = hipMalloc(&ptr_, bytes);
        if (e != hipSuccess) {
            ptr_ = nullptr;
            return hip_fail(e, "hipMalloc");
        }
        bytes_ = bytes;
        return RA_OK;
    }
    // Grow-only reuse (plan scratch).
    ra_status ensure(size_t bytes) {
        if (bytes <= bytes_) return RA_OK;
        return allocate(bytes);
    }
    template <typename T>
    ra_status upload(const std::vector<T>& v) {
        RA_TRY(allocate(v.size() * sizeof(T)));
        if (!v.empty()) {
            hipError_t e = hipMemcpy(ptr_, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice);
            if (e != hipSuccess) return hip_fail(e, "hipMemcpy H2D");
        }
        return RA_OK;
    }
    void reset() {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
    }
    template <typename T = void>
    T* get() const { return static_cast<T*>(ptr_); }
    size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Small host thread pool substitute: run f(i) for i in [0, n) on up to
// hardware_concurrency threads (plan builders; no OpenMP runtime needed).
void parallel_for(int64_t n, int64_t grain, const std::function<void(int64_t, int64_t)>& f);

// CSR_DIRECT launch (csr_kernels.hip).  resume = the fma chain of every output
// element continues from the value in C instead of 0 (C then holds the chain
// over an earlier column range of the same rows).
ra_status csr_direct_launch(const int32_t* d_rowptr, const int32_t* d_colind, const float* d_vals,
                            const float* d_B, float* d_C, int32_t M, int32_t K, int32_t N, int64_t nnz,
                            bool resume, hipStream_t st);

}  // namespace ra
