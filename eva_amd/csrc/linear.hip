// Single EXL3 linear, fp16 in / fp16 out (the config-1 layer).
//
// Reference: ELinear.forward -> LinearEXL3 (runtime/ds41/exl3_linear.py:97-131), kernel
// exl3_gemv_kernel.cuh:217-234 (input: fp16 x*suh, Hadamard, fp16), 295-459 (GEMV, fp16 C),
// 463-490 with hadamard_inner.cuh:93-147 (output Hadamard to fp16, fp16 product with svh).
// Two launches: rotate (+ counter reset), then GEMV with the output epilogue run by the last
// k-split to finish each 128-column chunk.
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
    float* part;       // [ks][rows][out]
    int* ctr;          // [out/128]
};

__global__ __launch_bounds__(256) void lin_rotate_kernel(LinParams p)
{
    const int lane = threadIdx.x & 63;
    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gtid < p.out / 128) p.ctr[gtid] = 0;
    const int item = gtid >> 6;
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
    dst[lane_col(lane, 0)] = f2h(v[0]);
    dst[lane_col(lane, 1)] = f2h(v[1]);
}

__global__ __launch_bounds__(256) void lin_gemv_kernel(LinParams p, const half_t* __restrict__ xr)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.ks) return;
    const int cg = wid / p.ks, ks = wid % p.ks;
    const int kt_n = p.in / 16;
    const int kt0 = kt_n * ks / p.ks, kt1 = kt_n * (ks + 1) / p.ks;
    gemv_dispatch_k(p.k2, p.trellis, p.out / 16, cg, kt0, kt1, xr, (size_t)p.in, k_iota, p.rows,
                    p.part + (size_t)ks * p.rows * p.out, (size_t)p.out);
    if (!arrive_last(p.ctr + cg, p.ks)) return;
    for (int m = 0; m < p.rows; ++m) {
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
}

int linear_ksplit(int rows, int in, int out)
{
    const int ncg = out / 128, kt_n = in / 16;
    int ks = (2048 + ncg - 1) / ncg;
    if (ks > kt_n / 4) ks = kt_n / 4;
    if (ks < 1) ks = 1;
    (void)rows;
    return ks;
}

size_t linear_workspace(int rows, int in, int out, size_t* off_part, size_t* off_ctr)
{
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const int ks = linear_ksplit(rows, in, out);
    size_t o = 0;
    o = al(o + (size_t)rows * in * 2);
    if (off_part) *off_part = o;
    o = al(o + (size_t)ks * rows * out * 4);
    if (off_ctr) *off_ctr = o;
    o = al(o + (size_t)(out / 128) * 4);
    return o;
}

int launch_linear(const void* x, int rows, int in, int out, const void* trellis, const void* suh,
                  const void* svh, int k2, void* y, void* ws, hipStream_t stream)
{
    LinParams p;
    size_t off_part, off_ctr;
    linear_workspace(rows, in, out, &off_part, &off_ctr);
    p.x = (const half_t*)x;
    p.rows = rows; p.in = in; p.out = out; p.k2 = k2;
    p.ks = linear_ksplit(rows, in, out);
    p.trellis = (const uint32_t*)trellis;
    p.suh = (const half_t*)suh;
    p.svh = (const half_t*)svh;
    p.y = (half_t*)y;
    p.xr = (half_t*)ws;
    p.part = (float*)((char*)ws + off_part);
    p.ctr = (int*)((char*)ws + off_ctr);
    {
        const int threads = rows * (in / 128) * 64;
        const int t = threads > out / 128 ? threads : out / 128;
        hipLaunchKernelGGL(lin_rotate_kernel, dim3((t + 255) / 256), dim3(256), 0, stream, p);
    }
    {
        const int waves = (out / 128) * p.ks;
        hipLaunchKernelGGL(lin_gemv_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p, (const half_t*)p.xr);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
