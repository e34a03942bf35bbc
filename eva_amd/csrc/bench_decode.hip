// Decode ALU ceiling: the rate at which gfx950 evaluates the EXL3 trellis decode of the GEMV
// (window funnels, MUL1 hashes, byte sums into fp16 pairs) with its matrix-core products (eight
// v_mfma_f32_4x4x4_16b_f16 per k-slice and row group) when nothing is loaded from memory. Every
// lane decodes one k-slice's 32 positions per iteration from register-resident words, which it
// then advances, exactly the per-weight instruction mix of the decode GEMV's inner loop for one
// row group (gemv_wave_m4, without its LDS activation reads). Bench.py divides the trellis
// bytes this rate implies into a GEMV's achieved bytes to say how close the GEMV is to the
// arithmetic bound, as opposed to the HBM bound.
//
// Read floor: the bytes of a decode GEMV launch streamed in that launch's shape without the
// decode, for the memory-side bound of the same launch (the HBM peak is reached only by long
// streams; a launch of tens of microseconds also pays its ramp and tail).
#include "evamx_gemv.hpp"
#include "evamx_internal.hpp"

namespace evamx {

template <int K2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void bench_decode_kernel(float* sink, int iters)
{
    using R = Rate<K2>;
    LaneWords<R::K> w;
#pragma unroll
    for (int i = 0; i <= R::K; ++i) w.b[i] = 0x9E3779B9u * (threadIdx.x + 7u * i + 1u) + blockIdx.x;
    const uint32_t sh = (threadIdx.x & 1) ? 0u : 16u;
    f32x4v_t acc[2] = {f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f}};
    const half4_t x = {(half_t)0.5f, (half_t)-0.25f, (half_t)0.125f, (half_t)1.0f};
    for (int it = 0; it < iters; ++it) {
        half2_t wp[16];
        decode_slice<K2>(w, sh, wp);
#pragma unroll
        for (int kg = 0; kg < 4; ++kg)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c] = __builtin_amdgcn_mfma_f32_4x4x4f16(x, m4_b(wp, c, kg), acc[c], 0, 0, 0);
#pragma unroll
        for (int i = 0; i <= R::K; ++i) w.b[i] += 0x7F4A7C15u * (i + 1);
    }
    // keep the work observable without storing per lane
    if (acc[0][0] + acc[1][1] == 1234.5f) sink[threadIdx.x] = acc[0][2];
}

// Wave w = (chain, cg), cg = w % ncg: the wave's 64 lanes read 16 bytes each from row
// chain * rows + i, at byte cg * 1024 of the row, for i < rows, with four rows in flight (the
// GEMV's prefetch depth and its non-temporal 16-byte loads); rows are row_u4 * 16 bytes apart.
__global__ __launch_bounds__(256) void bench_read_kernel(const u32x4* __restrict__ base, int ncg, int rows, int row_u4,
                                                         int n_waves, float* sink)
{
    const int w = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    if (w >= n_waves) return;
    const int lane = threadIdx.x & 63;
    const int cg = w % ncg, chain = w / ncg;
    const u32x4* q = base + (size_t)chain * rows * row_u4 + (size_t)cg * 64 + lane;
    uint32_t acc = 0;
    for (int i = 0; i < rows; i += 4) {
        u32x4 v[4];
#pragma unroll
        for (int d = 0; d < 4; ++d)
            v[d] = i + d < rows ? __builtin_nontemporal_load(q + (size_t)(i + d) * row_u4) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int d = 0; d < 4; ++d) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
    // keep the loads observable without storing per lane
    if (acc == 0x12345678u) sink[lane] = 1.0f;
}

void launch_bench_read(const void* base, int ncg, int rows, int n_waves, float* sink, hipStream_t stream)
{
    hipLaunchKernelGGL(bench_read_kernel, dim3((unsigned)((n_waves + 3) / 4)), dim3(256), 0, stream, (const u32x4*)base,
                       ncg, rows, ncg * 64, n_waves, sink);
}

int launch_bench_decode(int k2, int blocks, int iters, float* sink, hipStream_t stream)
{
    const dim3 g(blocks), b(256);
    switch (k2) {
        case 3: hipLaunchKernelGGL(bench_decode_kernel<3>, g, b, 0, stream, sink, iters); break;
        case 4: hipLaunchKernelGGL(bench_decode_kernel<4>, g, b, 0, stream, sink, iters); break;
        case 5: hipLaunchKernelGGL(bench_decode_kernel<5>, g, b, 0, stream, sink, iters); break;
        case 6: hipLaunchKernelGGL(bench_decode_kernel<6>, g, b, 0, stream, sink, iters); break;
        case 7: hipLaunchKernelGGL(bench_decode_kernel<7>, g, b, 0, stream, sink, iters); break;
        case 8: hipLaunchKernelGGL(bench_decode_kernel<8>, g, b, 0, stream, sink, iters); break;
        case 10: hipLaunchKernelGGL(bench_decode_kernel<10>, g, b, 0, stream, sink, iters); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
