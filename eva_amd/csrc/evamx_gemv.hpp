// Wave-level decode GEMV, Hadamard and completion-counter helpers shared by the MoE and the
// single-linear kernels.
//
// GEMV lane layout (wave64): lane = 8*i + q streams tile (kt, 8*cg + i) words q*K..q*K+K-1 with
// one vector load per k-slice and owns output columns 16i+q and 16i+q+8 of the 128-column group
// for all 16 k of the tile, so the k-loop needs no cross-lane reduction and a wave's 128 columns
// are exactly one Hadamard chunk. The 16 decoded k of a column pair up as (k, k+1) and meet the
// activation pairs (x[2m], x[2m+1]) in v_dot2_f32_f16 with fp32 accumulation.
#pragma once
#include "evamx_device.hpp"

namespace evamx {

__device__ __forceinline__ float h2f(half_t h) { return (float)h; }
__device__ __forceinline__ half_t f2h(float f) { return (half_t)f; }

// ---------------------------------------------------------------------------------------------
// Wave Hadamard over a 128-chunk held as two values per lane at element e = 16*(lane>>3) +
// 8*h + (lane&7): stages on e bits 0..6 in order (lane xor 1,2,4; in-lane; lane xor 8,16,32),
// which is the reference's order (hadamard_inner.cuh:17-44, exl3_moe_coop_kernel.cuh:131-147).

__device__ __forceinline__ int lane_col(int lane, int h) { return 16 * (lane >> 3) + 8 * h + (lane & 7); }

__device__ __forceinline__ void had128_lane(float& v0, float& v1, int lane)
{
#pragma unroll
    for (int b = 0; b < 3; ++b) {
        const int m = 1 << b;
        const bool up = (lane & m) != 0;
        v0 = bfly_x(v0, m, up);
        v1 = bfly_x(v1, m, up);
    }
    {
        const float a = v0, c = v1;
        v0 = a + c;
        v1 = a - c;
    }
#pragma unroll
    for (int b = 3; b < 6; ++b) {
        const int m = 1 << b;
        const bool up = (lane & m) != 0;
        v0 = bfly_x(v0, m, up);
        v1 = bfly_x(v1, m, up);
    }
    v0 *= R_SCALE;
    v1 *= R_SCALE;
}

// ---------------------------------------------------------------------------------------------
// Streaming loads.

typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// A lane's K words with one non-temporal 64/96/128-bit load (+1 dword at K=5).
template <int K>
__device__ __forceinline__ void load_words(LaneWords<K>& w, const uint32_t* p)
{
    if constexpr (K == 2) {
        const u32x2a v = __builtin_nontemporal_load((const u32x2a*)p);
        w.b[1] = v.x; w.b[2] = v.y;
    } else if constexpr (K == 3) {
        const u32x3a v = __builtin_nontemporal_load((const u32x3a*)p);
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z;
    } else {
        const u32x4a v = __builtin_nontemporal_load((const u32x4a*)p);
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z; w.b[4] = v.w;
#pragma unroll
        for (int i = 4; i < K; ++i) w.b[i + 1] = __builtin_nontemporal_load(p + i);
    }
}

// ---------------------------------------------------------------------------------------------
// Decode GEMV over one wave's k-range: acc[m][h] += sum_k A[slot_m][k] * W[k][col(lane,h)] for
// the tm (<= TM) rows slot_of[0..tm) of A (fp16, row stride a_stride elements).

template <int K, int TM>
__device__ __forceinline__ void gemv_wave(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                          const half_t* __restrict__ A, size_t a_stride, const int* slot_of,
                                          int tm, float (&acc)[TM][2])
{
    constexpr int TW = 8 * K;
    constexpr int PF = 4;
    const int lane = threadIdx.x & 63;
    const int q = lane & 7;
    const int src = (lane & ~7) | ((q + 7) & 7);
    const size_t slice = (size_t)nt_n * TW;
    const uint32_t* bp = trellis + (size_t)(cg * 8 + (lane >> 3)) * TW + q * K;

#pragma unroll
    for (int m = 0; m < TM; ++m) acc[m][0] = acc[m][1] = 0.0f;

    // Row offsets of the activation rows (wave-uniform: the loads below become scalar loads)
    uint32_t aoff[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m)
        aoff[m] = (uint32_t)__builtin_amdgcn_readfirstlane((m < tm ? slot_of[m] : slot_of[0]) * (int)(a_stride / 8));

    LaneWords<K> ring[PF];
#pragma unroll
    for (int d = 0; d < PF; ++d)
        if (kt0 + d < kt1) load_words<K>(ring[d], bp + (size_t)(kt0 + d) * slice);

    for (int kb = kt0; kb < kt1; kb += PF) {
#pragma unroll
        for (int d = 0; d < PF; ++d) {
            const int kt = kb + d;
            if (kt < kt1) {
            LaneWords<K> w = ring[d];
            if (kt + PF < kt1) load_words<K>(ring[d], bp + (size_t)(kt + PF) * slice);
            w.b[0] = __shfl(w.b[K], src, WAVE);
            half2_t wp[16];
#define EVAMX_DEC_UNIT(U)                                \
            wp[4 * U + 0] = lane_pair<K, 8 * U + 0>(w);  \
            wp[4 * U + 1] = lane_pair<K, 8 * U + 2>(w);  \
            wp[4 * U + 2] = lane_pair<K, 8 * U + 4>(w);  \
            wp[4 * U + 3] = lane_pair<K, 8 * U + 6>(w);
            EVAMX_DEC_UNIT(0)
            EVAMX_DEC_UNIT(1)
            EVAMX_DEC_UNIT(2)
            EVAMX_DEC_UNIT(3)
#undef EVAMX_DEC_UNIT
#pragma unroll
            for (int m = 0; m < TM; ++m) {
                if (m < tm) {
                const half2_t* xp = (const half2_t*)A + ((size_t)aoff[m] * 4 + (size_t)kt * 8);
                half2_t xa[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) xa[i] = xp[i];
                float a0 = acc[m][0], a1 = acc[m][1];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    a0 = dot2(wp[4 * u + 0], xa[u], a0);
                    a0 = dot2(wp[4 * u + 1], xa[u + 4], a0);
                    a1 = dot2(wp[4 * u + 2], xa[u], a1);
                    a1 = dot2(wp[4 * u + 3], xa[u + 4], a1);
                }
                acc[m][0] = a0;
                acc[m][1] = a1;
                }
            }
            }
        }
    }
}

// GEMV for a chunk of tm rows with the smallest template that fits; writes fp32 partials
// part[slot_of[m] * part_stride + column].
template <int K>
__device__ __forceinline__ void gemv_chunk(const uint32_t* trellis, int nt_n, int cg, int kt0, int kt1,
                                           const half_t* A, size_t a_stride, const int* slot_of, int tm,
                                           float* part, size_t part_stride)
{
    const int lane = threadIdx.x & 63;
    const int c0 = cg * 128 + lane_col(lane, 0), c1 = cg * 128 + lane_col(lane, 1);
#define EVAMX_RUN(TMV)                                                                        \
    {                                                                                         \
        float acc[TMV][2];                                                                    \
        gemv_wave<K, TMV>(trellis, nt_n, cg, kt0, kt1, A, a_stride, slot_of, tm, acc);        \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m) {                                     \
            if (m < tm) {                                                                     \
                float* dst = part + (size_t)slot_of[m] * part_stride;                         \
                dst[c0] = acc[m][0];                                                          \
                dst[c1] = acc[m][1];                                                          \
            }                                                                                 \
        }                                                                                     \
    }
    if (tm <= 1) EVAMX_RUN(1)
    else if (tm <= 2) EVAMX_RUN(2)
    else if (tm <= 4) EVAMX_RUN(4)
    else if (tm <= 8) EVAMX_RUN(8)
    else EVAMX_RUN(16)
#undef EVAMX_RUN
}

// Runtime rate (k2 = 2K) -> instantiated GEMV; integer rates 2..5.
__device__ __forceinline__ void gemv_dispatch_k(int k2, const uint32_t* trellis, int nt_n, int cg, int kt0, int kt1,
                                                const half_t* A, size_t a_stride, const int* slot_of, int tm,
                                                float* part, size_t part_stride)
{
    switch (k2) {
        case 4: gemv_chunk<2>(trellis, nt_n, cg, kt0, kt1, A, a_stride, slot_of, tm, part, part_stride); break;
        case 6: gemv_chunk<3>(trellis, nt_n, cg, kt0, kt1, A, a_stride, slot_of, tm, part, part_stride); break;
        case 8: gemv_chunk<4>(trellis, nt_n, cg, kt0, kt1, A, a_stride, slot_of, tm, part, part_stride); break;
        case 10: gemv_chunk<5>(trellis, nt_n, cg, kt0, kt1, A, a_stride, slot_of, tm, part, part_stride); break;
        default: break;
    }
}

// ---------------------------------------------------------------------------------------------
// Completion counter (exl3_moe_coop_kernel.cuh:549-559 semantics, per wave): every lane's stores
// are released at device scope, one lane arrives; true (wave-uniform) for the last of `expected`
// arrivals, which then acquires and may read the other waves' results.

__device__ __forceinline__ bool arrive_last(int* ctr, int expected)
{
    __threadfence();
    int old = 0;
    if ((threadIdx.x & 63) == 0) old = atomicAdd(ctr, 1);
    old = __shfl(old, 0, WAVE);
    const bool last = old == expected - 1;
    if (last) __threadfence();
    return last;
}

}  // namespace evamx
