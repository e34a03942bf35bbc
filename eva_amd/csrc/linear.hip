// Single EXL3 linear, fp16 in / fp16 out (the config-1 layer).
//
// Reference: ELinear.forward -> LinearEXL3 (runtime/ds41/exl3_linear.py:97-131), kernel
// exl3_gemv_kernel.cuh:217-234 (input: fp16 x*suh, Hadamard, fp16), 295-459 (GEMV, fp16 C),
// 463-490 with hadamard_inner.cuh:93-147 (output Hadamard to fp16, fp16 product with svh).
// Three launches: rotate, k-split decode GEMV into fp32 partials, and the output epilogue
// (the sum of the partials in fixed order, fp16 C, Hadamard, fp16 svh product).
#include "evamx_gemv.hpp"
#include "evamx_internal.hpp"

namespace evamx {

__constant__ int k_iota[16] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15};

struct LinParams {
    const half_t* x;
    int rows, in, out, k2, ks;
    const uint32_t* trellis;
    const half_t* suh;
    const half_t* svh;
    half_t* y;
    half_t* xr;        // [rows][in]
    float* xsum;       // [rows][in/128]
    float* part;       // [ks][rows][out]
};

__global__ __launch_bounds__(256) void lin_rotate_kernel(LinParams p)
{
    const int lane = threadIdx.x & 63;
    const int item = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nch = p.in / 128;
    if (item >= p.rows * nch) return;
    const int r = item / nch, c = item % nch;
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = c * 128 + lane_col(lane, h);
        v[h] = h2f(f2h(h2f(p.x[(size_t)r * p.in + col]) * h2f(p.suh[col])));   // fp16 product
    }
    had128_lane(v[0], v[1], lane);
    half_t* dst = p.xr + (size_t)r * p.in + c * 128;
    const half_t r0 = f2h(v[0]), r1 = f2h(v[1]);
    dst[lane_col(lane, 0)] = r0;
    dst[lane_col(lane, 1)] = r1;
    const float sum = wave_sum(h2f(r0) + h2f(r1));
    if (lane == 0) p.xsum[(size_t)r * nch + c] = sum;
}

template <int TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void lin_gemv_kernel(LinParams p, const half_t* __restrict__ xr)
{
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.ks) return;
    const int cg = __builtin_amdgcn_readfirstlane(wid / p.ks), ks = __builtin_amdgcn_readfirstlane(wid % p.ks);
    const int nch = p.in / 128;
    const int c0 = nch * ks / p.ks, c1 = nch * (ks + 1) / p.ks;
    gemv_dispatch_k<TMAX>(p.k2, p.trellis, p.out / 16, cg, c0, c1, GlobalRows{xr, (size_t)p.in, p.xsum, nch}, k_iota,
                    p.rows, p.part + (size_t)ks * p.rows * p.out, (size_t)p.out);
}

__global__ __launch_bounds__(256) void lin_epilogue_kernel(LinParams p)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.rows) return;
    const int m = wid / ncg, cg = wid % ncg;
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = cg * 128 + lane_col(lane, h);
        float acc = 0.0f;
        for (int q = 0; q < p.ks; ++q) acc += p.part[((size_t)q * p.rows + m) * p.out + col];
        v[h] = h2f(f2h(acc));                          // C in fp16
    }
    had128_lane(v[0], v[1], lane);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = cg * 128 + lane_col(lane, h);
        p.y[(size_t)m * p.out + col] = f2h(h2f(f2h(v[h])) * h2f(p.svh[col]));
    }
}

int linear_ksplit(int rows, int in, int out)
{
    const int ncg = out / 128, nch = in / 128;
    int ks = (4096 + ncg - 1) / ncg;
    if (ks > nch) ks = nch;
    if (ks < 1) ks = 1;
    (void)rows;
    return ks;
}

size_t linear_workspace(int rows, int in, int out, size_t* off_part, size_t* off_sum)
{
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const int ks = linear_ksplit(rows, in, out);
    size_t o = 0;
    o = al(o + (size_t)rows * in * 2);
    if (off_sum) *off_sum = o;
    o = al(o + (size_t)rows * (in / 128) * 4);
    if (off_part) *off_part = o;
    o = al(o + (size_t)ks * rows * out * 4);
    return o;
}

int launch_linear(const void* x, int rows, int in, int out, const void* trellis, const void* suh,
                  const void* svh, int k2, void* y, void* ws, hipStream_t stream)
{
    LinParams p;
    size_t off_part, off_sum;
    linear_workspace(rows, in, out, &off_part, &off_sum);
    p.x = (const half_t*)x;
    p.rows = rows; p.in = in; p.out = out; p.k2 = k2;
    p.ks = linear_ksplit(rows, in, out);
    p.trellis = (const uint32_t*)trellis;
    p.suh = (const half_t*)suh;
    p.svh = (const half_t*)svh;
    p.y = (half_t*)y;
    p.xr = (half_t*)ws;
    p.part = (float*)((char*)ws + off_part);
    p.xsum = (float*)((char*)ws + off_sum);
    {
        const int waves = rows * (in / 128);
        hipLaunchKernelGGL(lin_rotate_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p);
    }
    {
        const int waves = (out / 128) * p.ks;
        const dim3 grid((waves + 3) / 4);
        const half_t* xr = p.xr;
        switch (tmax_for(rows)) {
            case 1: hipLaunchKernelGGL(lin_gemv_kernel<1>, grid, dim3(256), 0, stream, p, xr); break;
            case 2: hipLaunchKernelGGL(lin_gemv_kernel<2>, grid, dim3(256), 0, stream, p, xr); break;
            case 4: hipLaunchKernelGGL(lin_gemv_kernel<4>, grid, dim3(256), 0, stream, p, xr); break;
            default: hipLaunchKernelGGL(lin_gemv_kernel<8>, grid, dim3(256), 0, stream, p, xr); break;
        }
    }
    {
        const int waves = (out / 128) * rows;
        hipLaunchKernelGGL(lin_epilogue_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
