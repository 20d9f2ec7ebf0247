/*
 * spmm_oracle.c — CPU restatement of the reference SpMM arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links or calls this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only as the checker.
 *
 * oracle_spmm_seq_f32  — the bit-level semantics of the reference CSR kernels:
 *     every output element is ONE fp32 accumulator updated as
 *     acc = fma(vals[p], B[col[p], n], acc) for p in CSR order.
 *     Reference: csr/csr_direct.cu:201-228 (subwarp kernel, nvcc --use_fast_math
 *     contracts `acc += a*b` to FMA, setup.py:52) and the small-row kernel of
 *     csr/ra_zero_overhead.cu:122-145.
 * oracle_spmm_f64      — the exact value in fp64 (error measurement).
 *
 * Built by oracle/Makefile with -ffp-contract=off so only the explicit fma()
 * calls fuse.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

void oracle_spmm_seq_f32(const int32_t* rowptr, const int32_t* colind, const float* vals,
                         const float* B, float* C, int32_t M, int32_t N)
{
    for (int32_t r = 0; r < M; ++r) {
        float* c = C + (int64_t)r * N;
        for (int32_t n = 0; n < N; ++n) c[n] = 0.0f;
        for (int32_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
            const float a = vals[p];
            const float* b = B + (int64_t)colind[p] * N;
            for (int32_t n = 0; n < N; ++n) c[n] = fmaf(a, b[n], c[n]);
        }
    }
}

void oracle_spmm_f64(const int32_t* rowptr, const int32_t* colind, const float* vals,
                     const float* B, double* C, int32_t M, int32_t N)
{
    for (int32_t r = 0; r < M; ++r) {
        double* c = C + (int64_t)r * N;
        for (int32_t n = 0; n < N; ++n) c[n] = 0.0;
        for (int32_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
            const double a = (double)vals[p];
            const float* b = B + (int64_t)colind[p] * N;
            for (int32_t n = 0; n < N; ++n) c[n] += a * (double)b[n];
        }
    }
}

/* Rows [r0, r1) only: used to bound the CPU baseline sample. */
void oracle_spmm_seq_f32_rows(const int32_t* rowptr, const int32_t* colind,
                              const float* vals, const float* B, float* C,
                              int32_t r0, int32_t r1, int32_t N)
{
    for (int32_t r = r0; r < r1; ++r) {
        float* c = C + (int64_t)(r - r0) * N;
        for (int32_t n = 0; n < N; ++n) c[n] = 0.0f;
        for (int32_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
            const float a = vals[p];
            const float* b = B + (int64_t)colind[p] * N;
            for (int32_t n = 0; n < N; ++n) c[n] = fmaf(a, b[n], c[n]);
        }
    }
}

/* Exact integer degree moments (sum of squares can exceed 2^53 only for
 * absurd graphs; int64 is exact up to 9.2e18). */
void oracle_degree_moments(const int32_t* rowptr, int32_t M, int64_t* nnz,
                           int64_t* sum_sq, int32_t* max_deg, int64_t* empty_rows)
{
    int64_t s2 = 0, e = 0;
    int32_t mx = 0;
    for (int32_t r = 0; r < M; ++r) {
        const int64_t d = (int64_t)rowptr[r + 1] - rowptr[r];
        s2 += d * d;
        if (d > mx) mx = (int32_t)d;
        if (d == 0) ++e;
    }
    *nnz = (int64_t)rowptr[M] - rowptr[0];
    *sum_sq = s2;
    *max_deg = mx;
    *empty_rows = e;
}
