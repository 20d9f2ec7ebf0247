// vendor_spmm.cpp — rocSPARSE SpMM as a measured comparator (not on the
// product path).  The reference's guardrail and the yardstick of its speed-up
// claims is the vendor library's CSR SpMM (cuSPARSE CSR_ALG2,
// bindings/ra_bindings.cpp:431-615); on MI355X the vendor library is
// rocSPARSE.  bench.py times every CSR algorithm rocSPARSE offers and reports
// the fastest.  C = A * B with alpha 1, beta 0, fp32, row-major B and C,
// int32 indices, the buffers the caller passes.
#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>

#include <cstdint>
#include <cstdio>
#include <new>

namespace {
thread_local char g_err[256] = "";

int fail(const char* what, int code) {
    std::snprintf(g_err, sizeof(g_err), "%s (status %d)", what, code);
    return code == 0 ? -1 : code;
}

struct VendorPlan {
    rocsparse_handle handle = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnmat_descr B = nullptr, C = nullptr;
    rocsparse_spmm_alg alg = rocsparse_spmm_alg_default;
    void* buffer = nullptr;
    size_t buffer_bytes = 0;
    ~VendorPlan() {
        if (buffer) (void)hipFree(buffer);
        if (A) rocsparse_destroy_spmat_descr(A);
        if (B) rocsparse_destroy_dnmat_descr(B);
        if (C) rocsparse_destroy_dnmat_descr(C);
        if (handle) rocsparse_destroy_handle(handle);
    }
};

rocsparse_status spmm(VendorPlan* p, rocsparse_spmm_stage stage) {
    const float one = 1.0f, zero = 0.0f;
    return rocsparse_spmm(p->handle, rocsparse_operation_none, rocsparse_operation_none, &one, p->A,
                          p->B, &zero, p->C, rocsparse_datatype_f32_r, p->alg, stage, &p->buffer_bytes,
                          p->buffer);
}
}  // namespace

extern "C" {

const char* ra_vendor_last_error(void) { return g_err; }

// alg: 0 default, 1 csr (row split, shared memory), 4 csr_row_split,
// 5 csr_nnz_split (merge), 9 csr_merge_path (rocsparse_spmm_alg values).
int ra_vendor_spmm_create(const int32_t* d_rowptr, const int32_t* d_colind, const float* d_vals,
                          const float* d_B, float* d_C, int32_t M, int32_t K, int32_t N, int64_t nnz,
                          int32_t alg, void* stream, void** out) {
    *out = nullptr;
    auto* p = new (std::nothrow) VendorPlan();
    if (!p) return fail("allocation", -1);
    p->alg = static_cast<rocsparse_spmm_alg>(alg);
    rocsparse_status s;
    if ((s = rocsparse_create_handle(&p->handle)) != rocsparse_status_success ||
        (s = rocsparse_set_stream(p->handle, static_cast<hipStream_t>(stream))) != rocsparse_status_success ||
        (s = rocsparse_create_csr_descr(&p->A, M, K, nnz, const_cast<int32_t*>(d_rowptr),
                                        const_cast<int32_t*>(d_colind), const_cast<float*>(d_vals),
                                        rocsparse_indextype_i32, rocsparse_indextype_i32,
                                        rocsparse_index_base_zero, rocsparse_datatype_f32_r)) !=
            rocsparse_status_success ||
        (s = rocsparse_create_dnmat_descr(&p->B, K, N, N, const_cast<float*>(d_B), rocsparse_datatype_f32_r,
                                          rocsparse_order_row)) != rocsparse_status_success ||
        (s = rocsparse_create_dnmat_descr(&p->C, M, N, N, d_C, rocsparse_datatype_f32_r,
                                          rocsparse_order_row)) != rocsparse_status_success ||
        (s = spmm(p, rocsparse_spmm_stage_buffer_size)) != rocsparse_status_success) {
        delete p;
        return fail("rocsparse set-up", s);
    }
    if (p->buffer_bytes > 0 && hipMalloc(&p->buffer, p->buffer_bytes) != hipSuccess) {
        delete p;
        return fail("hipMalloc of the rocsparse buffer", -1);
    }
    if ((s = spmm(p, rocsparse_spmm_stage_preprocess)) != rocsparse_status_success) {
        delete p;
        return fail("rocsparse preprocess", s);
    }
    *out = p;
    return 0;
}

// Runs on `stream` (the caller's current stream at this call, so C is written
// in order with the work that allocates and reads it).
int ra_vendor_spmm_run(void* plan, void* stream) {
    auto* p = static_cast<VendorPlan*>(plan);
    rocsparse_status s = rocsparse_set_stream(p->handle, static_cast<hipStream_t>(stream));
    if (s != rocsparse_status_success) return fail("rocsparse set stream", s);
    s = spmm(p, rocsparse_spmm_stage_compute);
    return s == rocsparse_status_success ? 0 : fail("rocsparse compute", s);
}

// Point the plan at another B and C of the same shapes (the analysis and
// buffer stay valid: they depend on A only).
int ra_vendor_spmm_set_dense(void* plan, const float* d_B, float* d_C) {
    auto* p = static_cast<VendorPlan*>(plan);
    rocsparse_status s;
    if ((s = rocsparse_dnmat_set_values(p->B, const_cast<float*>(d_B))) != rocsparse_status_success ||
        (s = rocsparse_dnmat_set_values(p->C, d_C)) != rocsparse_status_success)
        return fail("rocsparse set values", s);
    return 0;
}

void ra_vendor_spmm_destroy(void* plan) { delete static_cast<VendorPlan*>(plan); }

}  // extern "C"
