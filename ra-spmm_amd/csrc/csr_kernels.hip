// csr_kernels.hip — CSR family on 64-lane wavefronts (gfx950).
//
//   CSR_DIRECT         a lane group of G lanes owns one row; each lane keeps V
//                      packets (float4 when N % 4 == 0 and buffers are 16-byte
//                      aligned, float otherwise) of the output row, so one
//                      wave-wide dwordx4 load gathers 64/G whole B rows.
//                      (col, val) of a G-wide slice of the row are loaded
//                      coalesced, one per lane, and broadcast with ds_bpermute.
//   baseline           regime-free reference point: one wave per row, lanes
//                      stride over columns, scalar loads.
//   ZERO_OVERHEAD_CSR  one fused launch: hub chunks (256 nnz) first, then the
//                      degree-binned short rows; rows of up to 256 nonzeros
//                      keep one fma chain per element; chunks of rows longer
//                      than 256 write fp32 partials that a second launch sums
//                      in ascending chunk order (deterministic, no atomics).
//   features           exact integer degree moments (nnz, sum d^2, max d,
//                      empty rows): one launch up to 65,536 rows, two
//                      deterministic launches above; the result goes to
//                      mapped pinned host memory, which the host polls.
//
// Every output element of CSR_DIRECT, of the baseline and of ZO rows <= 256 is
// one fp32 accumulator updated by fma in CSR order, which is bit-identical to
// the reference per-lane accumulation (csr/csr_direct.cu:201-228).
#include <algorithm>
#include <cstdlib>
#include <chrono>
#include <mutex>

#include "ra_internal.hpp"
#include "zo_plan.hpp"

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;

// ZO bin thresholds (csr/ra_zero_overhead.cu:55-59).
using ra::kTiny;
using ra::kShort;
using ra::kMedium;
using ra::kChunk;
using ra::kSoleFlag;

// ------------------------------------------------------------------ packets
template <typename P> __device__ __forceinline__ P pzero();
template <> __device__ __forceinline__ float pzero<float>() { return 0.f; }
template <> __device__ __forceinline__ float4 pzero<float4>() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ __forceinline__ float pfma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ float4 pfma(float a, float4 b, float4 c) {
    return make_float4(__builtin_fmaf(a, b.x, c.x), __builtin_fmaf(a, b.y, c.y),
                       __builtin_fmaf(a, b.z, c.z), __builtin_fmaf(a, b.w, c.w));
}
__device__ __forceinline__ float padd(float a, float b) { return a + b; }
__device__ __forceinline__ float4 padd(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Streaming (non-temporal) accesses for data touched once: the CSR index and
// value streams and the C rows.  They then do not displace B rows that other
// waves are about to gather again from L2.
typedef float f32x4n __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ T load_once(const T* p, bool nt) {
    return nt ? __builtin_nontemporal_load(p) : *p;
}
__device__ __forceinline__ void store_once(float* p, float v, bool nt) {
    if (nt) __builtin_nontemporal_store(v, p);
    else *p = v;
}
__device__ __forceinline__ void store_once(float4* p, float4 v, bool nt) {
    if (nt) __builtin_nontemporal_store(f32x4n{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4n*>(p));
    else *p = v;
}

// Accumulate the nnz range [p0, p1) of one row into acc.  All G lanes of the
// group share the range; lane `sl` owns packet columns q[s] (q < 0: masked).
// Per output element the update order is p ascending, one fma per nonzero.
template <int G, int V, int U, typename P>
__device__ __forceinline__ void accumulate_range(const int32_t* __restrict__ colind,
                                                 const float* __restrict__ vals,
                                                 const P* __restrict__ Bp, int64_t ldp,
                                                 int p0, int p1, int sl, const int (&q)[V],
                                                 P (&acc)[V], bool nt) {
    static_assert(U <= G, "unroll deeper than the lane group");
    for (int base = p0; base < p1; base += G) {
        const int my = base + sl;
        int mc = 0;
        float mv = 0.f;
        if (my < p1) {
            mc = load_once(colind + my, nt);
            mv = load_once(vals + my, nt);
        }
        const int cnt = min(G, p1 - base);
        for (int j = 0; j < cnt; j += U) {
            int c[U];
            float a[U];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                c[k] = __shfl(mc, j + k, G);
                a[k] = __shfl(mv, j + k, G);
            }
            P b[U][V];
#pragma unroll
            for (int k = 0; k < U; ++k) {
#pragma unroll
                for (int s = 0; s < V; ++s) {
                    b[k][s] = (j + k < cnt && q[s] >= 0) ? Bp[(int64_t)c[k] * ldp + q[s]]
                                                        : pzero<P>();
                }
            }
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (j + k < cnt) {
#pragma unroll
                    for (int s = 0; s < V; ++s) acc[s] = pfma(a[k], b[k][s], acc[s]);
                }
            }
        }
    }
}

// As accumulate_range, with the (column, value) pairs of [p0, p1) already in
// LDS (s_col / s_val indexed from the chunk start): one broadcast LDS read per
// pair instead of a coalesced global load and a lane shuffle.
template <int G, int V, int U, typename P>
__device__ __forceinline__ void accumulate_lds(const int32_t* s_col, const float* s_val,
                                               const P* __restrict__ Bp, int64_t ldp, int p0, int p1,
                                               const int (&q)[V], P (&acc)[V]) {
    for (int p = p0; p < p1; p += U) {
        int c[U];
        float a[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            c[k] = p + k < p1 ? s_col[p + k] : 0;
            a[k] = p + k < p1 ? s_val[p + k] : 0.f;
        }
        P b[U][V];
#pragma unroll
        for (int k = 0; k < U; ++k)
#pragma unroll
            for (int s = 0; s < V; ++s)
                b[k][s] = (p + k < p1 && q[s] >= 0) ? Bp[(int64_t)c[k] * ldp + q[s]] : pzero<P>();
#pragma unroll
        for (int k = 0; k < U; ++k)
            if (p + k < p1) {
#pragma unroll
                for (int s = 0; s < V; ++s) acc[s] = pfma(a[k], b[k][s], acc[s]);
            }
    }
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// With remap on, XCD x runs a contiguous range of logical blocks, so rows that
// are close in the row order (and tend to share columns) share one L2.
__device__ __forceinline__ int64_t logical_block(bool remap) {
    const int64_t bid = blockIdx.x;
    if (!remap) return bid;
    const int64_t nb = gridDim.x, q = nb / 8, r = nb % 8;
    const int64_t x = bid % 8, k = bid / 8;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// Row block and column slice of this workgroup.  nslices > 0: a 1-D grid in
// which consecutive workgroups take consecutive column slices of the same
// rows; workgroups are dealt round-robin to the 8 XCDs, so with 8 % nslices
// == 0 every XCD gathers one column slice of B and its L2 holds that slice
// only.  nslices == 0: the slice is blockIdx.y (slices outermost).
__device__ __forceinline__ int64_t block_and_slice(bool remap, int nslices, int& slice) {
    if (nslices > 0) {
        slice = static_cast<int>(blockIdx.x % nslices);
        return blockIdx.x / nslices;
    }
    slice = blockIdx.y;
    return logical_block(remap);
}

// ---------------------------------------------------------------- CSR_DIRECT
template <int G, int V, int U, typename P>
__global__ __launch_bounds__(kBlock) void csr_rows_kernel(
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colind,
    const float* __restrict__ vals, const P* __restrict__ Bp, P* __restrict__ Cp,
    const int32_t* __restrict__ row_list, int64_t num_rows, int64_t ldp, int np, int remap,
    int nt, int resume, int nslices) {
    constexpr int RPW = kWave / G;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sub = lane / G;
    const int sl = lane % G;
    int slice;
    const int64_t idx = (block_and_slice(remap, nslices, slice) * kWavesPerBlock + wave) * RPW + sub;
    if (idx >= num_rows) return;  // whole lane groups leave together
    const int row = row_list ? row_list[idx] : static_cast<int>(idx);
    const int q0 = slice * (G * V);
    int q[V];
#pragma unroll
    for (int s = 0; s < V; ++s) {
        const int qq = q0 + sl + s * G;
        q[s] = qq < np ? qq : -1;
    }
    // resume: the fma chain continues from C (a later column range of the same
    // rows; storing and reloading the fp32 accumulator changes no bit).
    P acc[V];
#pragma unroll
    for (int s = 0; s < V; ++s)
        acc[s] = (resume && q[s] >= 0) ? Cp[(int64_t)row * ldp + q[s]] : pzero<P>();
    accumulate_range<G, V, U, P>(colind, vals, Bp, ldp, rowptr[row], rowptr[row + 1], sl, q, acc,
                                 nt != 0);
#pragma unroll
    for (int s = 0; s < V; ++s)
        if (q[s] >= 0) store_once(Cp + (int64_t)row * ldp + q[s], acc[s], nt != 0);
}

// ----------------------------------------------------------------- baseline
// One wave per row; lane covers columns lane + 64*i (i < 4) of a 256-column tile.
// T = float, or _Float16 for the precision-matched variant (A and B stored in
// fp16, products and sums in fp32).
template <typename T>
__global__ __launch_bounds__(kBlock) void csr_baseline_kernel(
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colind,
    const T* __restrict__ vals, const T* __restrict__ B, float* __restrict__ C,
    int M, int N) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= M) return;
    const int n0 = blockIdx.y * 256 + lane;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const int p1 = rowptr[row + 1];
    for (int p = rowptr[row]; p < p1; ++p) {
        const int c = colind[p];
        const float v = static_cast<float>(vals[p]);
        const T* b = B + (int64_t)c * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + 64 * i;
            if (n < N) acc[i] = __builtin_fmaf(v, static_cast<float>(b[n]), acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + 64 * i;
        if (n < N) C[(int64_t)row * N + n] = acc[i];
    }
}

// ---------------------------------------------------------- ZERO_OVERHEAD_CSR
// Waves [0, num_chunks) take one 256-nnz chunk each.  A sole chunk (a row of
// 65..256 nonzeros) is run by lane group 0 alone, one fma chain per element.
// A chunk of a longer row is split by the 64/G lane groups of the wave into
// contiguous parts that are summed in group order through LDS (with
// RA_ZO_SOLE_SPLIT=1 sole chunks are split the same way; measured no faster
// on C2 and C5).  Later waves take 64/G rows of the short-row list each.
template <int G, int V, int U, typename P>
__global__ __launch_bounds__(kBlock) void zo_fused_kernel(
    const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colind,
    const float* __restrict__ vals, const P* __restrict__ Bp, P* __restrict__ Cp,
    const int32_t* __restrict__ chunk_rows, const int32_t* __restrict__ chunk_starts,
    const int32_t* __restrict__ chunk_slot, int num_chunks, P* __restrict__ partials,
    const int32_t* __restrict__ short_rows, int64_t num_short, int64_t ldp, int np, int remap,
    int nt, int sole_split, int nslices, int lds_stage) {
    constexpr int RPW = kWave / G;
    __shared__ P red[kWavesPerBlock][(RPW > 1 ? RPW - 1 : 1) * G * V];
    __shared__ int s_col[kWavesPerBlock][kChunk];
    __shared__ float s_val[kWavesPerBlock][kChunk];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sub = lane / G;
    const int sl = lane % G;
    int slice;
    const int64_t gw = block_and_slice(remap, nslices, slice) * kWavesPerBlock + wave;
    const int q0 = slice * (G * V);
    int q[V];
#pragma unroll
    for (int s = 0; s < V; ++s) {
        const int qq = q0 + sl + s * G;
        q[s] = qq < np ? qq : -1;
    }
    P acc[V];
#pragma unroll
    for (int s = 0; s < V; ++s) acc[s] = pzero<P>();

    if (gw < num_chunks) {
        const uint32_t tag = static_cast<uint32_t>(chunk_rows[gw]);
        const int row = static_cast<int>(tag & ~kSoleFlag);
        const int cs = chunk_starts[gw];
        const int ce = min(cs + kChunk, rowptr[row + 1]);
        if (lds_stage) {
            // The chunk's (column, value) pairs go to LDS first, in one
            // coalesced pass by the whole wave (RA_ZO_LDS_STAGE=0: loaded G at a
            // time and shuffled, as for the short rows).
            for (int i = lane; i < ce - cs; i += kWave) {
                s_col[wave][i] = load_once(colind + cs + i, nt != 0);
                s_val[wave][i] = load_once(vals + cs + i, nt != 0);
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
            __builtin_amdgcn_wave_barrier();
        }
        if ((tag & kSoleFlag) && !sole_split) {
            // A sole chunk (a row of 65..256 nonzeros) is one lane group's
            // single fma chain per element, as for the short rows: the same
            // bits as CSR_DIRECT (csr/ra_zero_overhead.cu:246-262).
            if (sub != 0) return;
            if (lds_stage) accumulate_lds<G, V, U, P>(s_col[wave], s_val[wave], Bp, ldp, 0, ce - cs, q, acc);
            else accumulate_range<G, V, U, P>(colind, vals, Bp, ldp, cs, ce, sl, q, acc, nt != 0);
#pragma unroll
            for (int s = 0; s < V; ++s)
                if (q[s] >= 0) store_once(Cp + (int64_t)row * ldp + q[s], acc[s], nt != 0);
            return;
        }
        constexpr int L = kChunk / RPW;
        const int a = min(cs + sub * L, ce);
        const int b = min(a + L, ce);
        if (lds_stage) accumulate_lds<G, V, U, P>(s_col[wave], s_val[wave], Bp, ldp, a - cs, b - cs, q, acc);
        else accumulate_range<G, V, U, P>(colind, vals, Bp, ldp, a, b, sl, q, acc, nt != 0);
        if constexpr (RPW > 1) {
            if (sub > 0) {
#pragma unroll
                for (int s = 0; s < V; ++s) red[wave][((sub - 1) * V + s) * G + sl] = acc[s];
            }
            // LDS writes of groups 1.. must land before group 0 reads them
            // (same wave: a workgroup-scope fence orders the LDS accesses).
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
            __builtin_amdgcn_wave_barrier();
            if (sub == 0) {
                for (int h = 1; h < RPW; ++h) {
#pragma unroll
                    for (int s = 0; s < V; ++s)
                        acc[s] = padd(acc[s], red[wave][((h - 1) * V + s) * G + sl]);
                }
            }
        }
        if (sub == 0) {
            const int slot = chunk_slot[gw];
            P* dst = (tag & kSoleFlag) ? Cp + (int64_t)row * ldp : partials + (int64_t)slot * ldp;
#pragma unroll
            for (int s = 0; s < V; ++s)
                if (q[s] >= 0) store_once(dst + q[s], acc[s], nt != 0);
        }
        return;
    }
    const int64_t idx = (gw - num_chunks) * RPW + sub;
    if (idx >= num_short) return;
    const int row = short_rows[idx];
    accumulate_range<G, V, U, P>(colind, vals, Bp, ldp, rowptr[row], rowptr[row + 1], sl, q, acc,
                                 nt != 0);
#pragma unroll
    for (int s = 0; s < V; ++s)
        if (q[s] >= 0) store_once(Cp + (int64_t)row * ldp + q[s], acc[s], nt != 0);
}

// Deterministic merge: C[row] = ((slot0 + slot1) + slot2) + ... per element.
// One thread per (split row, packet); rows are packed np to a workgroup so
// narrow N does not idle lanes, and slots are loaded 16 at a time so a hub
// row's chain of ~200 partials costs ~13 memory round trips, not ~200.  The
// additions stay in ascending slot order.
template <typename P>
__global__ __launch_bounds__(kBlock) void zo_merge_kernel(
    const int32_t* __restrict__ split_rows, const int32_t* __restrict__ split_off,
    const P* __restrict__ partials, P* __restrict__ Cp, int64_t ldp, int np, int nrows) {
    constexpr int D = 16;
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t r = t / np;
    if (r >= nrows) return;
    const int qq = static_cast<int>(t - r * np);
    const int o0 = split_off[r], o1 = split_off[r + 1];
    P acc = partials[(int64_t)o0 * ldp + qq];
    int o = o0 + 1;
    for (; o + D <= o1; o += D) {
        P x[D];
#pragma unroll
        for (int i = 0; i < D; ++i) x[i] = partials[(int64_t)(o + i) * ldp + qq];
#pragma unroll
        for (int i = 0; i < D; ++i) acc = padd(acc, x[i]);
    }
    for (; o < o1; ++o) acc = padd(acc, partials[(int64_t)o * ldp + qq]);
    Cp[(int64_t)split_rows[r] * ldp + qq] = acc;
}

// ------------------------------------------------------------------ features
constexpr int kMomentBlocks = 512;

__device__ __forceinline__ long long wave_sum_ll(long long v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
    return v;
}

// Block sums of (d^2, empty rows) and the block max of d over the rows
// blockIdx.x * BS + threadIdx.x + k * gridDim.x * BS; valid in thread 0.
template <int BS>
__device__ __forceinline__ void block_moments(const int32_t* __restrict__ rowptr, int M,
                                              long long& sq_out, int& mx_out, long long& em_out) {
    constexpr int W = BS / kWave;
    __shared__ long long s_sq[W], s_em[W];
    __shared__ int s_mx[W];
    long long sq = 0, em = 0;
    int mx = 0;
    // Eight rows per thread per step, their loads issued together (a strided
    // loop with one row per step waits one memory latency per row).
    constexpr int kU = 8;
    const int stride = gridDim.x * BS;
    for (int r0 = blockIdx.x * BS + threadIdx.x; r0 < M; r0 += kU * stride) {
        int lo[kU], hi[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int r = r0 + u * stride;
            lo[u] = r < M ? rowptr[r] : 0;
            hi[u] = r < M ? rowptr[r + 1] : 0;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (r0 + u * stride >= M) break;
            const long long d = (long long)hi[u] - lo[u];
            sq += d * d;
            em += (d == 0);
            mx = max(mx, (int)d);
        }
    }
    sq = wave_sum_ll(sq);
    em = wave_sum_ll(em);
    mx = wave_max_i(mx);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        s_sq[wave] = sq;
        s_em[wave] = em;
        s_mx[wave] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        sq = em = 0;
        mx = 0;
        for (int w = 0; w < W; ++w) {
            sq += s_sq[w];
            em += s_em[w];
            mx = max(mx, s_mx[w]);
        }
        sq_out = sq;
        mx_out = mx;
        em_out = em;
    }
}

// out (mapped pinned host memory) = {nnz, sum d^2, max d, empty rows, seq}:
// the four values, a system-scope fence, then the call's sequence number, so a
// host that reads seq back sees the values of this call.
__device__ __forceinline__ void publish_moments(long long* out, long long nnz, long long sq, int mx,
                                                long long em, long long seq) {
    out[0] = nnz;
    out[1] = sq;
    out[2] = mx;
    out[3] = em;
    __threadfence_system();
    __hip_atomic_store(&out[4], seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A small matrix in one block of 1024 lanes, which writes the result itself.
__global__ __launch_bounds__(1024) void degree_moments_one(const int32_t* __restrict__ rowptr, int M,
                                                           long long* __restrict__ out, long long seq) {
    long long sq = 0, em = 0;
    int mx = 0;
    block_moments<1024>(rowptr, M, sq, mx, em);
    if (threadIdx.x == 0) publish_moments(out, (long long)rowptr[M] - rowptr[0], sq, mx, em, seq);
}

// Per-block partials: [block][0] = sum d^2, [1] = max d, [2] = empty rows.
__global__ __launch_bounds__(kBlock) void degree_moments_partial(const int32_t* __restrict__ rowptr, int M,
                                                                 long long* __restrict__ part) {
    long long sq = 0, em = 0;
    int mx = 0;
    block_moments<kBlock>(rowptr, M, sq, mx, em);
    if (threadIdx.x != 0) return;
    part[blockIdx.x * 3 + 0] = sq;
    part[blockIdx.x * 3 + 1] = mx;
    part[blockIdx.x * 3 + 2] = em;
}

// Single block: out = {nnz, sum d^2, max d, empty rows} from the partials.
__global__ __launch_bounds__(kBlock) void degree_moments_final(
    const long long* __restrict__ part, int nparts, const int32_t* __restrict__ rowptr, int M,
    long long* __restrict__ out, long long seq) {
    __shared__ long long s_sq[kWavesPerBlock], s_em[kWavesPerBlock];
    __shared__ int s_mx[kWavesPerBlock];
    long long sq = 0, em = 0;
    int mx = 0;
    for (int i = threadIdx.x; i < nparts; i += kBlock) {
        sq += part[i * 3 + 0];
        mx = max(mx, (int)part[i * 3 + 1]);
        em += part[i * 3 + 2];
    }
    sq = wave_sum_ll(sq);
    em = wave_sum_ll(em);
    mx = wave_max_i(mx);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        s_sq[wave] = sq;
        s_em[wave] = em;
        s_mx[wave] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        long long a = 0, e = 0;
        int m = 0;
        for (int w = 0; w < kWavesPerBlock; ++w) {
            a += s_sq[w];
            e += s_em[w];
            m = max(m, s_mx[w]);
        }
        publish_moments(out, (long long)rowptr[M] - rowptr[0], a, m, e, seq);
    }
}

// Rows up to which one block reduces the whole rowptr (one launch; a second,
// dependent launch costs ~7 us of queue latency on MI355X).
constexpr int kMomentOneBlockRows = 1 << 16;

// Per-device reduction buffers, allocated once and kept for the process.
struct MomentBuffers {
    long long* part = nullptr;
    long long* host = nullptr;       // pinned, mapped: the kernels write the result here
    long long* host_dev = nullptr;   // its device address
    long long seq = 0;               // sequence number of the last call
};
std::mutex g_moment_mutex;
MomentBuffers g_moment[64];

// --------------------------------------------------------------- dispatch
struct LaneShape {
    int G, V, U;
};

// Tuning knobs, read once per process: RA_CSR_LANES forces the lane-group
// width (4..64), RA_CSR_UNROLL the gathers in flight per lane (4 or 8),
// RA_XCD_REMAP=0 turns the XCD-contiguous block order of CSR_DIRECT off
// (RA_ZO_XCD_REMAP=1 turns it on for ZERO_OVERHEAD_CSR, where it piles the hub
// chunks onto one XCD), RA_CSR_STREAMING=0 turns the non-temporal hints off,
// RA_CSR_COLTILE=c processes the columns in passes of c elements (the grid's
// slowest dimension), so each pass gathers only a c-column slice of B;
// RA_ZO_SOLE_SPLIT=1 splits sole ZO chunks over the wave's lane groups;
// RA_ZO_LDS_STAGE=0 turns off the LDS staging of the chunks' (column, value)
// pairs; RA_CSR_SLICE=c sets CSR_DIRECT's XCD-dealt column slice (0 off;
// default 128 columns at N >= 256 when the unsliced grid has < 2^16 waves).
struct CsrTuning {
    int lanes = 0, unroll = 4, remap = 1, zo_remap = 0, nt = 1, coltile = 0, sole_split = 0, xslice = 0,
        zo_slice = -1, lds_stage = 1, csr_slice = -1;
    CsrTuning() {
        if (const char* e = std::getenv("RA_CSR_SLICE")) csr_slice = std::atoi(e);
        if (const char* e = std::getenv("RA_ZO_LDS_STAGE")) lds_stage = std::atoi(e) != 0;
        if (const char* e = std::getenv("RA_ZO_SLICE")) zo_slice = std::atoi(e);
        if (const char* e = std::getenv("RA_CSR_XSLICE")) xslice = std::atoi(e) != 0;
        if (const char* e = std::getenv("RA_ZO_SOLE_SPLIT")) sole_split = std::atoi(e) != 0;
        if (const char* e = std::getenv("RA_CSR_COLTILE")) coltile = std::atoi(e);
        if (const char* e = std::getenv("RA_CSR_LANES")) lanes = std::atoi(e);
        if (const char* e = std::getenv("RA_CSR_UNROLL")) unroll = std::atoi(e) >= 8 ? 8 : 4;
        if (const char* e = std::getenv("RA_XCD_REMAP")) remap = std::atoi(e) != 0;
        if (const char* e = std::getenv("RA_ZO_XCD_REMAP")) zo_remap = std::atoi(e) != 0;
        if (const char* e = std::getenv("RA_CSR_STREAMING")) nt = std::atoi(e) != 0;
    }
};
const CsrTuning& tuning() {
    static const CsrTuning t;
    return t;
}

// Lane-group shape from the number of packets per row (per column pass).
LaneShape pick_shape(int np, int packet_elems, int slice_elems = 0) {
    const CsrTuning& t = tuning();
    if (slice_elems > 0) np = std::min(np, std::max(1, slice_elems / packet_elems));
    else if (t.coltile > 0) np = std::min(np, std::max(1, t.coltile / packet_elems));
    int G;
    if (t.lanes >= 4 && t.lanes <= 64 && (t.lanes & (t.lanes - 1)) == 0) G = t.lanes;
    else G = np <= 4 ? 4 : np <= 8 ? 8 : np <= 16 ? 16 : np <= 32 ? 32 : 64;
    int V = (np + G - 1) / G;
    V = V <= 1 ? 1 : V <= 2 ? 2 : 4;
    const int U = std::min(G, t.unroll);
    return {G, V, U};
}

// True when grid.x * grid.y work-groups of kBlock lanes fit one grid dimension.
inline bool fold_fits(dim3 grid) {
    return static_cast<uint64_t>(grid.x) * grid.y * kBlock <= 0xFFFFFFFFull;
}

template <typename P>
ra_status launch_csr_rows(const LaneShape& sh, dim3 grid, hipStream_t st, const int32_t* rowptr,
                          const int32_t* colind, const float* vals, const P* B, P* C,
                          const int32_t* row_list, int64_t num_rows, int64_t ldp, int np, int resume,
                          bool xcd_slices) {
    const int remap = tuning().remap, nt = tuning().nt;
    int nslices = 0;
    // Folding the column slices into grid.x is legal only while the folded
    // grid stays below 2^32 work-items (grid.x * blockDim on AMD); beyond
    // that the 2-D grid (one slice per grid.y) is kept.
    if (xcd_slices && grid.y > 1 && fold_fits(grid)) {
        nslices = static_cast<int>(grid.y);
        grid = dim3(grid.x * grid.y, 1);
    }
#define RA_ROWS_CASE(g, v, u)                                                               \
    if (sh.G == g && sh.V == v && sh.U == u) {                                              \
        csr_rows_kernel<g, v, u, P><<<grid, kBlock, 0, st>>>(rowptr, colind, vals, B, C,    \
                                                             row_list, num_rows, ldp, np,   \
                                                             remap, nt, resume, nslices);   \
        RA_LAUNCH_CHECK("csr_rows_kernel");                                                 \
        return RA_OK;                                                                       \
    }
#define RA_ROWS_G(g, u) RA_ROWS_CASE(g, 1, u) RA_ROWS_CASE(g, 2, u) RA_ROWS_CASE(g, 4, u)
    RA_ROWS_G(4, 4)
    RA_ROWS_G(8, 4)
    RA_ROWS_G(8, 8)
    RA_ROWS_G(16, 4)
    RA_ROWS_G(16, 8)
    RA_ROWS_G(32, 4)
    RA_ROWS_G(32, 8)
    RA_ROWS_G(64, 4)
    RA_ROWS_G(64, 8)
#undef RA_ROWS_G
#undef RA_ROWS_CASE
    return ra::fail(RA_ERR_INTERNAL, "csr_rows: no lane shape");
}

template <typename P>
ra_status launch_zo(const LaneShape& sh, dim3 grid, hipStream_t st, const int32_t* rowptr,
                    const int32_t* colind, const float* vals, const P* B, P* C,
                    const int32_t* chunk_rows, const int32_t* chunk_starts,
                    const int32_t* chunk_slot, int num_chunks, P* partials,
                    const int32_t* short_rows, int64_t num_short, int64_t ldp, int np,
                    bool xcd_slices) {
    const int remap = tuning().zo_remap, nt = tuning().nt, sole_split = tuning().sole_split;
    int nslices = 0;
    if (xcd_slices && grid.y > 1 && fold_fits(grid)) {  // same 2^32 work-item bound
        nslices = static_cast<int>(grid.y);
        grid = dim3(grid.x * grid.y, 1);
    }
#define RA_ZO_CASE(g, v, u)                                                                  \
    if (sh.G == g && sh.V == v && sh.U == u) {                                               \
        zo_fused_kernel<g, v, u, P><<<grid, kBlock, 0, st>>>(                                \
            rowptr, colind, vals, B, C, chunk_rows, chunk_starts, chunk_slot, num_chunks,    \
            partials, short_rows, num_short, ldp, np, remap, nt, sole_split, nslices,        \
            tuning().lds_stage);                                                             \
        RA_LAUNCH_CHECK("zo_fused_kernel");                                                  \
        return RA_OK;                                                                        \
    }
#define RA_ZO_G(g, u) RA_ZO_CASE(g, 1, u) RA_ZO_CASE(g, 2, u) RA_ZO_CASE(g, 4, u)
    RA_ZO_G(4, 4)
    RA_ZO_G(8, 4)
    RA_ZO_G(8, 8)
    RA_ZO_G(16, 4)
    RA_ZO_G(16, 8)
    RA_ZO_G(32, 4)
    RA_ZO_G(32, 8)
    RA_ZO_G(64, 4)
    RA_ZO_G(64, 8)
#undef RA_ZO_G
#undef RA_ZO_CASE
    return ra::fail(RA_ERR_INTERNAL, "zo: no lane shape");
}

ra_status check_spmm_args(const void* rowptr, const void* colind, const void* vals,
                          const void* B, const void* C, int32_t M, int32_t K, int32_t N,
                          int64_t nnz) {
    if (M < 0 || K < 0 || N < 0 || nnz < 0)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "negative dimension");
    if (M > 0 && !rowptr) return ra::fail(RA_ERR_INVALID_ARGUMENT, "rowptr is NULL");
    if (nnz > 0 && (!colind || !vals)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "colind/vals NULL");
    if (M > 0 && N > 0 && !C) return ra::fail(RA_ERR_INVALID_ARGUMENT, "C is NULL");
    if (nnz > 0 && N > 0 && !B) return ra::fail(RA_ERR_INVALID_ARGUMENT, "B is NULL");
    if (nnz > INT32_MAX) return ra::fail(RA_ERR_UNSUPPORTED, "nnz exceeds int32 indexing");
    return RA_OK;
}

}  // namespace

// ============================================================ ZO plan object

namespace ra {

ra_status csr_direct_launch(const int32_t* d_rowptr, const int32_t* d_colind, const float* d_vals,
                            const float* d_B, float* d_C, int32_t M, int32_t K, int32_t N, int64_t nnz,
                            bool resume, hipStream_t st) {
    RA_TRY(check_spmm_args(d_rowptr, d_colind, d_vals, d_B, d_C, M, K, N, nnz));
    if (M == 0 || N == 0) return RA_OK;
    const bool vec = (N % 4 == 0) && ra::aligned16(d_B) && ra::aligned16(d_C);
    const int np = vec ? N / 4 : N;
    // Wide rows of a small matrix: 128-column slices dealt to the XCDs, as
    // ZERO_OVERHEAD_CSR does, so that fewer than 2^16 waves (about 64 per CU)
    // become 2-4x as many, each with a shorter chain of dependent gathers.
    // On larger matrices the slices only re-read A per slice (config 3 at
    // N=512: 1.91 -> 2.18 ms), so they stay off there.
    int cslice = tuning().csr_slice;
    if (cslice < 0) {
        const LaneShape whole = pick_shape(np, vec ? 4 : 1);
        const int64_t waves = (static_cast<int64_t>(M) + kWave / whole.G - 1) / (kWave / whole.G);
        cslice = (vec && N >= 256 && waves < (int64_t{1} << 16)) ? 128 : 0;
    }
    const LaneShape sh = pick_shape(np, vec ? 4 : 1, cslice);
    const bool deal = cslice > 0 || tuning().xslice;
    const int rows_per_block = kWavesPerBlock * (kWave / sh.G);
    dim3 grid((M + rows_per_block - 1) / rows_per_block, (np + sh.G * sh.V - 1) / (sh.G * sh.V));
    if (vec)
        return launch_csr_rows<float4>(sh, grid, st, d_rowptr, d_colind, d_vals,
                                       reinterpret_cast<const float4*>(d_B),
                                       reinterpret_cast<float4*>(d_C), nullptr, M, np, np, resume ? 1 : 0,
                                       deal);
    return launch_csr_rows<float>(sh, grid, st, d_rowptr, d_colind, d_vals, d_B, d_C,
                                  nullptr, M, np, np, resume ? 1 : 0, deal);
}

}  // namespace ra

// partials: the split chunks' slot buffer ([num_split_chunks][N] fp32), or
// NULL to use (and grow) the plan's own.
static ra_status zo_run(ra_zo_plan* plan, const int32_t* d_rowptr, const int32_t* d_colind,
                 const float* d_vals, const float* d_B, float* d_C, int32_t N, int32_t stage,
                 float* partials, hipStream_t st) {
    if (stage < 0 || stage > 2) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: stage must be 0, 1 or 2");
    if (!plan) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: plan is NULL");
    const int32_t M = plan->info.M;
    RA_TRY(check_spmm_args(d_rowptr, d_colind, d_vals, d_B, d_C, M, plan->info.K, N, 0));
    if (M == 0 || N == 0) return RA_OK;
    const bool vec = (N % 4 == 0) && ra::aligned16(d_B) && ra::aligned16(d_C);
    const int np = vec ? N / 4 : N;
    // Wide rows are cut into 128-column slices dealt to the XCDs (each XCD's
    // L2 then holds half or less of every gathered B row).
    const int zslice = tuning().zo_slice >= 0 ? tuning().zo_slice : (vec && N >= 256 ? 128 : 0);
    const LaneShape sh = pick_shape(np, vec ? 4 : 1, zslice);
    if (plan->info.num_split_chunks > 0 && !partials) {
        RA_TRY(plan->partials.ensure((size_t)plan->info.num_split_chunks * N * sizeof(float)));
        partials = plan->partials.get<float>();
    }
    const int RPW = kWave / sh.G;
    const int64_t waves = plan->info.num_chunks + (plan->num_short_total + RPW - 1) / RPW;
    const int tiles = (np + sh.G * sh.V - 1) / (sh.G * sh.V);
    if (waves > 0 && stage != 2) {
        dim3 grid((waves + kWavesPerBlock - 1) / kWavesPerBlock, tiles);
        ra_status s;
        if (vec)
            s = launch_zo<float4>(sh, grid, st, d_rowptr, d_colind, d_vals,
                                  reinterpret_cast<const float4*>(d_B), reinterpret_cast<float4*>(d_C),
                                  plan->chunk_rows, plan->chunk_starts,
                                  plan->chunk_slot, plan->info.num_chunks,
                                  reinterpret_cast<float4*>(partials), plan->short_rows,
                                  plan->num_short_total, np, np, zslice > 0);
        else
            s = launch_zo<float>(sh, grid, st, d_rowptr, d_colind, d_vals, d_B, d_C,
                                 plan->chunk_rows, plan->chunk_starts,
                                 plan->chunk_slot, plan->info.num_chunks,
                                 partials, plan->short_rows,
                                 plan->num_short_total, np, np, zslice > 0);
        RA_TRY(s);
    }
    if (plan->info.num_split_rows > 0 && stage != 1) {
        const int64_t threads = (int64_t)plan->info.num_split_rows * np;
        const unsigned grid = static_cast<unsigned>((threads + kBlock - 1) / kBlock);
        if (vec)
            zo_merge_kernel<float4><<<grid, kBlock, 0, st>>>(
                plan->split_rows, plan->split_off,
                reinterpret_cast<float4*>(partials), reinterpret_cast<float4*>(d_C), np, np,
                plan->info.num_split_rows);
        else
            zo_merge_kernel<float><<<grid, kBlock, 0, st>>>(
                plan->split_rows, plan->split_off,
                partials, d_C, np, np, plan->info.num_split_rows);
        RA_LAUNCH_CHECK("zo_merge_kernel");
    }
    return RA_OK;
}

namespace ra {
ra_status zo_run_with_partials(ra_zo_plan* plan, const int32_t* d_rowptr, const int32_t* d_colind,
                               const float* d_vals, const float* d_B, float* d_C, int32_t N, float* partials,
                               hipStream_t st) {
    return zo_run(plan, d_rowptr, d_colind, d_vals, d_B, d_C, N, 0, partials, st);
}
}  // namespace ra

extern "C" {

ra_status ra_spmm_csr_direct(const int32_t* d_rowptr, const int32_t* d_colind,
                             const float* d_vals, const float* d_B, float* d_C, int32_t M,
                             int32_t K, int32_t N, int64_t nnz, ra_stream_t stream) {
    return ra::csr_direct_launch(d_rowptr, d_colind, d_vals, d_B, d_C, M, K, N, nnz, false,
                                 reinterpret_cast<hipStream_t>(stream));
}

ra_status ra_spmm_csr_baseline(const int32_t* d_rowptr, const int32_t* d_colind,
                               const float* d_vals, const float* d_B, float* d_C, int32_t M,
                               int32_t K, int32_t N, int64_t nnz, ra_stream_t stream) {
    RA_TRY(check_spmm_args(d_rowptr, d_colind, d_vals, d_B, d_C, M, K, N, nnz));
    if (M == 0 || N == 0) return RA_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    dim3 grid((M + kWavesPerBlock - 1) / kWavesPerBlock, (N + 255) / 256);
    csr_baseline_kernel<float><<<grid, kBlock, 0, st>>>(d_rowptr, d_colind, d_vals, d_B, d_C, M, N);
    RA_LAUNCH_CHECK("csr_baseline_kernel");
    return RA_OK;
}

ra_status ra_spmm_csr_baseline_f16(const int32_t* d_rowptr, const int32_t* d_colind,
                                   const uint16_t* d_vals_h, const uint16_t* d_B_h, float* d_C, int32_t M,
                                   int32_t K, int32_t N, int64_t nnz, ra_stream_t stream) {
    RA_TRY(check_spmm_args(d_rowptr, d_colind, d_vals_h, d_B_h, d_C, M, K, N, nnz));
    if (M == 0 || N == 0) return RA_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    dim3 grid((M + kWavesPerBlock - 1) / kWavesPerBlock, (N + 255) / 256);
    csr_baseline_kernel<_Float16><<<grid, kBlock, 0, st>>>(d_rowptr, d_colind,
                                                           reinterpret_cast<const _Float16*>(d_vals_h),
                                                           reinterpret_cast<const _Float16*>(d_B_h), d_C, M, N);
    RA_LAUNCH_CHECK("csr_baseline_kernel_f16");
    return RA_OK;
}

// --------------------------------------------------------------- features
ra_status ra_features_device(const int32_t* d_rowptr, int32_t M, int32_t K, int32_t N,
                             ra_stream_t stream, ra_features* out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: out is NULL");
    if (M < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: M < 0");
    if (M == 0) return ra_features_from_moments(0, K, N, 0, 0, 0, 0, out);
    if (!d_rowptr) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: rowptr is NULL");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int dev = 0;
    RA_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return ra::fail(RA_ERR_UNSUPPORTED, "features: device id >= 64");
    MomentBuffers* mb = &g_moment[dev];
    // One feature pass at a time per process: the buffers are per device and
    // the wait below reads them back (a pass takes ~15 us).
    std::lock_guard<std::mutex> lock(g_moment_mutex);
    if (!mb->part) {
        RA_HIP_TRY(hipMalloc(&mb->part, sizeof(long long) * 3 * kMomentBlocks));
        RA_HIP_TRY(hipHostMalloc(&mb->host, sizeof(long long) * 5,
                                 hipHostMallocMapped | hipHostMallocCoherent));
        mb->host[4] = 0;
        RA_HIP_TRY(hipHostGetDevicePointer(reinterpret_cast<void**>(&mb->host_dev), mb->host, 0));
    }
    // The result goes straight to mapped pinned host memory (no copy).
    const long long seq = ++mb->seq;
    if (M <= kMomentOneBlockRows) {
        degree_moments_one<<<1, 1024, 0, st>>>(d_rowptr, M, mb->host_dev, seq);
        RA_LAUNCH_CHECK("degree_moments_one");
    } else {
        const int blocks = std::max(2, std::min(kMomentBlocks, (M + kBlock * 4 - 1) / (kBlock * 4)));
        degree_moments_partial<<<blocks, kBlock, 0, st>>>(d_rowptr, M, mb->part);
        RA_LAUNCH_CHECK("degree_moments_partial");
        degree_moments_final<<<1, kBlock, 0, st>>>(mb->part, blocks, d_rowptr, M, mb->host_dev, seq);
        RA_LAUNCH_CHECK("degree_moments_final");
    }
    // Wait by polling the sequence number the last kernel publishes (a
    // stream synchronisation adds ~5 us to a ~15 us call).  After ~200 us
    // (earlier work queued on the stream, or a failed kernel) fall back to
    // the synchronisation, which returns any launch or execution error.
    long long* flag = mb->host + 4;
    bool seen = false;
    const auto t0 = std::chrono::steady_clock::now();
    for (int spin = 0; !seen; ++spin) {
        seen = __atomic_load_n(flag, __ATOMIC_ACQUIRE) == seq;
        if (!seen && (spin & 1023) == 1023 &&
            std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200))
            break;
    }
    if (!seen) {
        RA_HIP_TRY(hipStreamSynchronize(st));
        if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq)
            return ra::fail(RA_ERR_INTERNAL, "features: the reduction did not publish its result");
    }
    return ra_features_from_moments(M, K, N, mb->host[0], mb->host[1],
                                    static_cast<int32_t>(mb->host[2]), mb->host[3], out);
}

// --------------------------------------------------------------------- ZO
ra_status ra_zo_bins_host(const int32_t* h_rowptr, int32_t M, int32_t K, int32_t* small_rows,
                          int32_t* chunk_rows, int32_t* chunk_starts, int32_t* empty_rows,
                          ra_zo_info* info) {
    // Binning of csr/ra_zero_overhead.cu:331-358 (same thresholds and chunk
    // layout); the small list is tiny, short, medium, each ascending.
    if (!info) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: info is NULL");
    if (M < 0 || (M > 0 && !h_rowptr)) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: bad rowptr");
    ra_zo_info z{};
    z.M = M;
    z.K = K;
    int64_t max_long = 0;
    for (int32_t i = 0; i < M; ++i) {
        const int64_t d = (int64_t)h_rowptr[i + 1] - h_rowptr[i];
        if (d < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: rowptr not monotone");
        if (d == 0) ++z.num_empty;
        else if (d <= kTiny) ++z.num_tiny;
        else if (d <= kShort) ++z.num_short;
        else if (d <= kMedium) ++z.num_medium;
        else {
            ++z.num_long;
            max_long = std::max(max_long, d);
            const int nch = static_cast<int>((d + kChunk - 1) / kChunk);
            z.num_chunks += nch;
            if (nch == 1) ++z.num_sole_chunks;
            else {
                ++z.num_split_rows;
                z.num_split_chunks += nch;
            }
        }
    }
    z.num_small = z.num_tiny + z.num_short + z.num_medium;
    z.max_long_chunks = static_cast<int32_t>((max_long + kChunk - 1) / kChunk);
    int64_t t = 0, s = z.num_tiny, m = (int64_t)z.num_tiny + z.num_short, c = 0, e = 0;
    for (int32_t i = 0; i < M; ++i) {
        const int32_t start = h_rowptr[i];
        const int64_t d = (int64_t)h_rowptr[i + 1] - start;
        if (d == 0) {
            if (empty_rows) empty_rows[e] = i;
            ++e;
        } else if (d <= kTiny) {
            if (small_rows) small_rows[t] = i;
            ++t;
        } else if (d <= kShort) {
            if (small_rows) small_rows[s] = i;
            ++s;
        } else if (d <= kMedium) {
            if (small_rows) small_rows[m] = i;
            ++m;
        } else {
            const bool sole = d <= kChunk;
            for (int64_t off = 0; off < d; off += kChunk) {
                if (chunk_rows) chunk_rows[c] = sole ? static_cast<int32_t>(uint32_t(i) | kSoleFlag) : i;
                if (chunk_starts) chunk_starts[c] = static_cast<int32_t>(start + off);
                ++c;
            }
        }
    }
    z.plan_bytes = (int64_t)sizeof(int32_t) *
                   ((int64_t)z.num_small + z.num_empty + 3LL * z.num_chunks + 2LL * z.num_split_rows + 1);
    *info = z;
    return RA_OK;
}

ra_status ra_zo_plan_create(const int32_t* h_rowptr, int32_t M, int32_t K, ra_zo_plan** out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: out is NULL");
    *out = nullptr;
    ra_zo_info z{};
    RA_TRY(ra_zo_bins_host(h_rowptr, M, K, nullptr, nullptr, nullptr, nullptr, &z));
    std::vector<int32_t> small(z.num_small), empty(z.num_empty), crow(z.num_chunks),
        cstart(z.num_chunks);
    RA_TRY(ra_zo_bins_host(h_rowptr, M, K, small.data(), crow.data(), cstart.data(), empty.data(), &z));
    // Short-row list handed to the kernel: empty rows first (they only write
    // zeros), then the bin-ordered small rows.
    std::vector<int32_t> short_rows;
    short_rows.reserve(empty.size() + small.size());
    short_rows.insert(short_rows.end(), empty.begin(), empty.end());
    short_rows.insert(short_rows.end(), small.begin(), small.end());
    // Partial slots of split rows: consecutive and ascending per row.
    std::vector<int32_t> slot(z.num_chunks, -1), split_rows, split_off{0};
    int32_t next = 0;
    for (int32_t c = 0; c < z.num_chunks;) {
        const uint32_t tag = static_cast<uint32_t>(crow[c]);
        if (tag & kSoleFlag) {
            ++c;
            continue;
        }
        const int32_t row = crow[c];
        split_rows.push_back(row);
        while (c < z.num_chunks && crow[c] == row) slot[c++] = next++;
        split_off.push_back(next);
    }
    auto plan = new (std::nothrow) ra_zo_plan();
    if (!plan) return ra::fail(RA_ERR_OUT_OF_MEMORY, "zo: plan allocation");
    ra_status s = RA_OK;
    (void)hipGetDevice(&plan->device);
    auto up = [](int32_t* d, const std::vector<int32_t>& v) -> ra_status {
        if (!v.empty()) RA_HIP_TRY(hipMemcpy(d, v.data(), v.size() * sizeof(int32_t), hipMemcpyHostToDevice));
        return RA_OK;
    };
    if ((s = plan->carve(static_cast<int64_t>(short_rows.size()), z.num_chunks, z.num_split_rows)) == RA_OK &&
        (s = up(plan->chunk_rows, crow)) == RA_OK && (s = up(plan->chunk_starts, cstart)) == RA_OK &&
        (s = up(plan->chunk_slot, slot)) == RA_OK && (s = up(plan->short_rows, short_rows)) == RA_OK &&
        (s = up(plan->split_rows, split_rows)) == RA_OK && (s = up(plan->split_off, split_off)) == RA_OK) {
        plan->info = z;
        plan->num_short_total = static_cast<int64_t>(short_rows.size());
        *out = plan;
        return RA_OK;
    }
    delete plan;
    return s;
}

ra_status ra_zo_plan_run(ra_zo_plan* plan, const int32_t* d_rowptr, const int32_t* d_colind,
                         const float* d_vals, const float* d_B, float* d_C, int32_t N,
                         ra_stream_t stream) {
    return ra_zo_plan_run_stage(plan, d_rowptr, d_colind, d_vals, d_B, d_C, N, 0, stream);
}

ra_status ra_zo_plan_run_stage(ra_zo_plan* plan, const int32_t* d_rowptr,
                               const int32_t* d_colind, const float* d_vals, const float* d_B,
                               float* d_C, int32_t N, int32_t stage, ra_stream_t stream) {
    return zo_run(plan, d_rowptr, d_colind, d_vals, d_B, d_C, N, stage, nullptr,
                  reinterpret_cast<hipStream_t>(stream));
}

ra_status ra_zo_plan_get_info(const ra_zo_plan* plan, ra_zo_info* info) {
    if (!plan || !info) return ra::fail(RA_ERR_INVALID_ARGUMENT, "zo: NULL argument");
    *info = plan->info;
    return RA_OK;
}

void ra_zo_plan_destroy(ra_zo_plan* plan) { delete plan; }

}  // extern "C"
