// gather_probe.hip — a measurement probe, not on the product path: the rate
// at which the GPU gathers whole B rows in a given order, with nothing else
// to do.  Run over a CSR's column indices it is the data-movement ceiling of
// any row-gathering SpMM on that matrix (every nonzero gathers its B row
// once, in CSR order), without the row structure, the fmas or C.
//
// A lane group of G = row packets lanes (float4 packets, G <= 64) gathers one
// B row per index; each wave walks a contiguous range of the index stream
// (`span` indices per group), loads the indices coalesced, broadcasts them
// with lane shuffles and keeps 4 gathers in flight per lane, like the CSR
// kernels.  Each lane adds what it gathered and writes one float4 at the end,
// so the write traffic is negligible.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

template <int G>
__global__ __launch_bounds__(kBlock) void gather_rows_probe(const float4* __restrict__ B, int64_t ldp,
                                                            const int32_t* __restrict__ idx, int64_t n,
                                                            float4* __restrict__ out, int span) {
    constexpr int RPW = kWave / G;
    const int lane = threadIdx.x & (kWave - 1);
    const int sub = lane / G;
    const int sl = lane % G;
    const int64_t group = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / kWave * RPW + sub;
    const int64_t p0 = group * span;
    const int64_t p1 = p0 + span < n ? p0 + span : n;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t base = p0; base < p1; base += G) {
        const int mine = base + sl < p1 ? __builtin_nontemporal_load(idx + base + sl) : 0;
        const int cnt = static_cast<int>(p1 - base < G ? p1 - base : G);
        for (int j = 0; j < cnt; j += 4) {
            float4 b[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int c = __shfl(mine, j + k, G);
                b[k] = j + k < cnt ? B[(int64_t)c * ldp + sl] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc.x += b[k].x;
                acc.y += b[k].y;
                acc.z += b[k].z;
                acc.w += b[k].w;
            }
        }
    }
    out[(int64_t)blockIdx.x * kBlock + threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// Gathers B[idx[i], 0:4*packets] for i < n.  B: fp32, row stride ldp float4
// packets; packets in {4, 8, 16, 32, 64} (N = 16..256 columns); each lane
// group walks `span` consecutive indices.  out must hold
// ra_probe_out_elems(n, packets, span) float4 (that function returns -1 for
// packets or span out of range).  Returns 0, or -1 on bad arguments.
static bool probe_args_ok(int32_t packets, int32_t span) {
    return (packets == 4 || packets == 8 || packets == 16 || packets == 32 || packets == 64) && span >= 1;
}

int64_t ra_probe_out_elems(int64_t n, int32_t packets, int32_t span) {
    if (!probe_args_ok(packets, span)) return -1;
    const int64_t groups = (n + span - 1) / span;
    const int64_t rpw = kWave / packets;
    const int64_t waves = (groups + rpw - 1) / rpw;
    return (waves + 3) / 4 * kBlock;
}

int ra_probe_gather(const float* B, int64_t ldp, int32_t packets, const int32_t* idx, int64_t n, int32_t span,
                    float* out, void* stream) {
    if (!probe_args_ok(packets, span)) return -1;
    if (n <= 0) return 0;
    const int64_t blocks = ra_probe_out_elems(n, packets, span) / kBlock;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float4* B4 = reinterpret_cast<const float4*>(B);
    float4* o = reinterpret_cast<float4*>(out);
    switch (packets) {
        case 4: gather_rows_probe<4><<<blocks, kBlock, 0, st>>>(B4, ldp, idx, n, o, span); break;
        case 8: gather_rows_probe<8><<<blocks, kBlock, 0, st>>>(B4, ldp, idx, n, o, span); break;
        case 16: gather_rows_probe<16><<<blocks, kBlock, 0, st>>>(B4, ldp, idx, n, o, span); break;
        case 32: gather_rows_probe<32><<<blocks, kBlock, 0, st>>>(B4, ldp, idx, n, o, span); break;
        case 64: gather_rows_probe<64><<<blocks, kBlock, 0, st>>>(B4, ldp, idx, n, o, span); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
