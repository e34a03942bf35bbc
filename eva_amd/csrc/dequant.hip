// EXL3 trellis -> fp16 W[k][n] (bit-exact decode).
//
// Reference: exl3_dq.cuh:15-31 (windows), codebook.cuh:86-99 (MUL1), the tile layout of
// exl3_moe_coop_kernel.cuh:377,404 and the fragment map of rocm/ptx_rocm.cuh:11-14.
#include "evamx_device.hpp"
#include "evamx_internal.hpp"

namespace evamx {

// Lane-structured decode (the same code the decode GEMV runs): one wave = 8 consecutive tiles
// of one k-slice; lane = (tile i, q) owns columns q, q+8 of tile i for all 16 k.
template <int K>
__global__ __launch_bounds__(256) void dequant_lane_kernel(const uint32_t* __restrict__ trellis,
                                                           int kt_n, int nt_n, half_t* __restrict__ w)
{
    constexpr int TW = 8 * K;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int groups = (nt_n + 7) / 8;
    const int kt = wave / groups;
    if (kt >= kt_n) return;
    const int nt = (wave % groups) * 8 + (lane >> 3);
    const int q = lane & 7;
    const bool ok = nt < nt_n;

    LaneWords<K> lw;
    const uint32_t* tp = trellis + ((size_t)kt * nt_n + (ok ? nt : 0)) * TW + q * K;
#pragma unroll
    for (int i = 0; i < K; ++i) lw.b[i + 1] = tp[i];
    const int src = (lane & ~7) | ((q + 7) & 7);
    lw.b[0] = __shfl(lw.b[K], src, WAVE);
    if (!ok) return;

    const size_t n_out = (size_t)nt_n * 16;
    half_t* base = w + (size_t)(16 * kt) * n_out + 16 * nt + q;
#define EVAMX_STORE_UNIT(U)                                                        \
    {                                                                              \
        const half2_t p0 = lane_pair<K, 8 * U + 0>(lw);                            \
        const half2_t p1 = lane_pair<K, 8 * U + 2>(lw);                            \
        const half2_t p2 = lane_pair<K, 8 * U + 4>(lw);                            \
        const half2_t p3 = lane_pair<K, 8 * U + 6>(lw);                            \
        base[(size_t)(2 * U + 0) * n_out] = p0.x;                                  \
        base[(size_t)(2 * U + 1) * n_out] = p0.y;                                  \
        base[(size_t)(2 * U + 8) * n_out] = p1.x;                                  \
        base[(size_t)(2 * U + 9) * n_out] = p1.y;                                  \
        base[(size_t)(2 * U + 0) * n_out + 8] = p2.x;                              \
        base[(size_t)(2 * U + 1) * n_out + 8] = p2.y;                              \
        base[(size_t)(2 * U + 8) * n_out + 8] = p3.x;                              \
        base[(size_t)(2 * U + 9) * n_out + 8] = p3.y;                              \
    }
    EVAMX_STORE_UNIT(0)
    EVAMX_STORE_UNIT(1)
    EVAMX_STORE_UNIT(2)
    EVAMX_STORE_UNIT(3)
#undef EVAMX_STORE_UNIT
}

// Scalar decode, any rate (k2 = 2K; half rates b+0.5 included): one thread per position.
__global__ __launch_bounds__(256) void dequant_scalar_kernel(const uint32_t* __restrict__ trellis,
                                                             int kt_n, int nt_n, int k2, half_t* __restrict__ w)
{
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t tiles = (size_t)kt_n * nt_n;
    if (gid >= tiles * 256) return;
    const size_t tile = gid >> 8;
    const int p = (int)(gid & 255);
    const int tw = 4 * k2;
    const uint32_t* tp = trellis + tile * tw;
    long end;
    if (!(k2 & 1)) end = (long)(p + 1) * (k2 / 2);
    else {
        const int b = k2 / 2, b2 = 2 * b + 1;
        end = (p & 1) ? (long)((p + 1) / 2) * b2 : (long)(p / 2) * b2 + b;
    }
    end += 32L * tw;
    const int i0 = (int)(((end - 16) / 32) % tw);
    const int i1 = (int)(((end - 1) / 32) % tw);
    const int s = (int)(((end - 1) / 32 + 1) * 32 - end);
    const uint32_t state = (uint32_t)((((uint64_t)tp[i0] << 32) | tp[i1]) >> s) & 0xffffu;
    const int lane = p >> 3, j = p & 7, g = lane >> 2, t = lane & 3;
    const int k = 2 * t + (j & 1) + 8 * ((j >> 1) & 1);
    const int n = g + 8 * (j >> 2);
    const size_t kt = tile / nt_n, nt = tile % nt_n;
    w[(16 * kt + k) * ((size_t)nt_n * 16) + 16 * nt + n] = mul1_one(state);
}

int launch_dequant(const void* trellis, int in, int out, int k2, void* w, bool scalar, hipStream_t stream)
{
    const int kt_n = in / 16, nt_n = out / 16;
    const uint32_t* t = (const uint32_t*)trellis;
    half_t* o = (half_t*)w;
    if (!scalar && !(k2 & 1) && k2 >= 4 && k2 <= 10) {
        const int waves = kt_n * ((nt_n + 7) / 8);
        const int blocks = (waves + 3) / 4;
        switch (k2 / 2) {
            case 2: hipLaunchKernelGGL(dequant_lane_kernel<2>, dim3(blocks), dim3(256), 0, stream, t, kt_n, nt_n, o); break;
            case 3: hipLaunchKernelGGL(dequant_lane_kernel<3>, dim3(blocks), dim3(256), 0, stream, t, kt_n, nt_n, o); break;
            case 4: hipLaunchKernelGGL(dequant_lane_kernel<4>, dim3(blocks), dim3(256), 0, stream, t, kt_n, nt_n, o); break;
            case 5: hipLaunchKernelGGL(dequant_lane_kernel<5>, dim3(blocks), dim3(256), 0, stream, t, kt_n, nt_n, o); break;
        }
    } else {
        const size_t threads = (size_t)kt_n * nt_n * 256;
        hipLaunchKernelGGL(dequant_scalar_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                           t, kt_n, nt_n, k2, o);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
