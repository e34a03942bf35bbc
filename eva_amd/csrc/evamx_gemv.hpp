// Wave-level decode GEMV and Hadamard helpers shared by the MoE and the single-linear kernels.
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
    v0 = bfly_x<1>(v0, lane);  v1 = bfly_x<1>(v1, lane);
    v0 = bfly_x<2>(v0, lane);  v1 = bfly_x<2>(v1, lane);
    v0 = bfly_x<4>(v0, lane);  v1 = bfly_x<4>(v1, lane);
    {
        const float a = v0, c = v1;
        v0 = a + c;
        v1 = a - c;
    }
    v0 = bfly_x<8>(v0, lane);  v1 = bfly_x<8>(v1, lane);
    v0 = bfly_x<16>(v0, lane); v1 = bfly_x<16>(v1, lane);
    v0 = bfly_x<32>(v0, lane); v1 = bfly_x<32>(v1, lane);
    v0 *= R_SCALE;
    v1 *= R_SCALE;
}

// ---------------------------------------------------------------------------------------------
// Streaming loads.

typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// Global-address-space view of a pointer. Loads through a generic pointer become flat loads,
// which also count against the LDS/scalar counter: every wait for a scalar activation load
// would then drain the whole weight prefetch ring.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const void* p)
{
    return (const __attribute__((address_space(1))) T*)p;
}

// A lane's K words with one non-temporal 64/96/128-bit global load (+1 dword at K=5).
template <int K>
__device__ __forceinline__ void load_words(LaneWords<K>& w, const uint32_t* p)
{
    if constexpr (K == 2) {
        const u32x2a v = __builtin_nontemporal_load(gptr<u32x2a>(p));
        w.b[1] = v.x; w.b[2] = v.y;
    } else if constexpr (K == 3) {
        const u32x3a v = __builtin_nontemporal_load(gptr<u32x3a>(p));
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z;
    } else {
        const u32x4a v = __builtin_nontemporal_load(gptr<u32x4a>(p));
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z; w.b[4] = v.w;
#pragma unroll
        for (int i = 4; i < K; ++i) w.b[i + 1] = __builtin_nontemporal_load(gptr<uint32_t>(p + i));
    }
}

// ---------------------------------------------------------------------------------------------
// Activation rows of a GEMV chunk: row m holds the k-vector of slot slot_of[m], read through
// wave-uniform addresses (scalar loads), together with its per-128-chunk sums (fp32) that the
// affine codebook map needs.

struct GlobalRows {
    const half_t* A;
    size_t stride;          // elements per row
    const float* sums;      // [row][chunk] sums of the fp16 row values over 128-element chunks
    int sums_stride;        // chunks per row
};

// ---------------------------------------------------------------------------------------------
// Decode GEMV over one wave's k-range [16*kt0, 16*kt1): acc[m][h] = sum_k X[m][k] * h_k,
// h_k = 1024 + bytesum of the weight at (k, col(lane, h)) (see mul1_hpair).

// The previous word of a lane's tile run: lane (l & ~7) | ((l - 1) & 7)'s last word. DPP row
// rotations within rows of 16 lanes: rotate by 1 serves lanes with l % 8 != 0, rotate by 9 the
// first lane of each group of 8 (no LDS round trip, unlike a bpermute).
__device__ __forceinline__ uint32_t prev_word(uint32_t v, int lane)
{
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xf, 0xf, false);   // row_ror:1
    const uint32_t r9 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x129, 0xf, 0xf, false);   // row_ror:9
    return (lane & 7) ? r1 : r9;
}

// Weight prefetch depth (k-slices in flight per wave): deeper for narrow chunks, whose loop
// body is short; wide chunks keep register pressure in check.
template <int TM>
constexpr int prefetch_depth() { return TM <= 2 ? 7 : 4; }

template <int K, int TM>
__device__ __forceinline__ void gemv_wave(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                          const GlobalRows& src, const uint32_t (&aoff)[TM], int tm, float (&acc)[TM][2])
{
    constexpr int TW = 8 * K;
    constexpr int PF = prefetch_depth<TM>();
    const int lane = threadIdx.x & 63;
    const int q = lane & 7;
    const size_t slice = (size_t)nt_n * TW;
    const uint32_t* bp = trellis + (size_t)(cg * 8 + (lane >> 3)) * TW + q * K;

#pragma unroll
    for (int m = 0; m < TM; ++m) acc[m][0] = acc[m][1] = 0.0f;

    // Prefetch ring: the row PF slices ahead, clamped to the wave's last row so that the steady
    // state needs no branch and never reads outside the matrix (the clamped reloads hit cache).
    LaneWords<K> ring[PF];
    const int last = kt1 - 1;
#pragma unroll
    for (int d = 0; d < PF; ++d) load_words<K>(ring[d], bp + (size_t)min(kt0 + d, last) * slice);

    // Narrow chunks load the next slice's activations (wave-uniform, scalar loads) one step
    // ahead, so their latency hides behind a decode instead of stalling every step.
    constexpr bool XPF = TM <= 2;
    half2_t xa[TM][8];
    auto load_x = [&](half2_t (&dst)[TM][8], int kt) {
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m < tm) {
                const half2_t* xp = (const half2_t*)src.A + ((size_t)aoff[m] * 4 + (size_t)kt * 8);
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[m][i] = xp[i];
            }
        }
    };
    if constexpr (XPF) load_x(xa, kt0);

    // Decode the slot, then refill the same registers with the slice PF ahead (issuing the load
    // before the decode would keep two copies of the slot live and make the compiler rotate
    // registers through moves that wait for every load in flight), then the dot products.
    auto step = [&](int kt, LaneWords<K>& w) {
        half2_t xn[TM][8];
        if constexpr (XPF) load_x(xn, min(kt + 1, last));
        w.b[0] = prev_word(w.b[K], lane);
        half2_t wp[16];
#define EVAMX_DEC_UNIT(U)                                \
        wp[4 * U + 0] = lane_hpair<K, 8 * U + 0>(w);     \
        wp[4 * U + 1] = lane_hpair<K, 8 * U + 2>(w);     \
        wp[4 * U + 2] = lane_hpair<K, 8 * U + 4>(w);     \
        wp[4 * U + 3] = lane_hpair<K, 8 * U + 6>(w);
        EVAMX_DEC_UNIT(0)
        EVAMX_DEC_UNIT(1)
        EVAMX_DEC_UNIT(2)
        EVAMX_DEC_UNIT(3)
#undef EVAMX_DEC_UNIT
        const int pre = __builtin_amdgcn_readfirstlane(min(kt + PF, last));
        load_words<K>(w, bp + (size_t)pre * slice);
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m < tm) {
                if constexpr (!XPF) {
                    const half2_t* xp = (const half2_t*)src.A + ((size_t)aoff[m] * 4 + (size_t)kt * 8);
#pragma unroll
                    for (int i = 0; i < 8; ++i) xa[m][i] = xp[i];
                }
                float a0 = acc[m][0], a1 = acc[m][1];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    a0 = dot2(wp[4 * u + 0], xa[m][u], a0);
                    a0 = dot2(wp[4 * u + 1], xa[m][u + 4], a0);
                    a1 = dot2(wp[4 * u + 2], xa[m][u], a1);
                    a1 = dot2(wp[4 * u + 3], xa[m][u + 4], a1);
                }
                acc[m][0] = a0;
                acc[m][1] = a1;
            }
            // wide chunks: keep at most four tokens' activations (32 SGPRs) live at a time
            if constexpr (TM >= 8)
                if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (XPF) {
#pragma unroll
            for (int m = 0; m < TM; ++m)
#pragma unroll
                for (int i = 0; i < 8; ++i) xa[m][i] = xn[m][i];
        }
        // keep the next step's scalar activation loads out of this one (register pressure)
        __builtin_amdgcn_sched_barrier(0);
    };

    int kt = kt0;
    for (; kt + PF <= kt1; kt += PF) {
#pragma unroll
        for (int d = 0; d < PF; ++d) step(kt + d, ring[d]);
    }
#pragma unroll
    for (int d = 0; d < PF - 1; ++d)
        if (kt + d < kt1) step(kt + d, ring[d]);
}

// GEMV for a chunk of tm rows over the 128-element k-chunks [c0, c1) with the smallest
// template that fits; writes fp32 partials part[slot_of[m] * part_stride + column] =
// sum_k x_k w_k = 0x1eee * sum_k x_k h_k + 0xc931 * sum_k x_k.
// Only the row variants up to TMAX are compiled in, so a launch for narrow chunks is not
// register-allocated for the widest one. A chunk of more than TMAX rows (possible only when
// given routes repeat an expert within a token) is processed TMAX rows at a time.
template <int K, int TMAX>
__device__ __forceinline__ void gemv_chunk(const uint32_t* trellis, int nt_n, int cg, int c0, int c1,
                                           const GlobalRows& src, const int* slot_of, int tm, float* part,
                                           size_t part_stride)
{
    const int lane = threadIdx.x & 63;
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#define EVAMX_RUN(TMV)                                                                          \
    {                                                                                           \
        uint32_t aoff[TMV];                                                                     \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m)                                         \
            aoff[m] = (uint32_t)__builtin_amdgcn_readfirstlane((m < tr ? so[m] : so[0]) *        \
                                                               (int)(src.stride / 8));          \
        float acc[TMV][2];                                                                      \
        gemv_wave<K, TMV>(trellis, nt_n, cg, 8 * c0, 8 * c1, src, aoff, tr, acc);               \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m) {                                       \
            if (m < tr) {                                                                       \
                const int row = so[m];                                                          \
                const float* sp = src.sums + (size_t)row * src.sums_stride;                     \
                float xs = 0.0f;                                                                \
                for (int c = c0; c < c1; ++c) xs += sp[c];                                      \
                float* dst = part + (size_t)row * part_stride;                                  \
                dst[col0] = MUL1_K_INV * acc[m][0] + MUL1_K_BIAS * xs;                          \
                dst[col1] = MUL1_K_INV * acc[m][1] + MUL1_K_BIAS * xs;                          \
            }                                                                                   \
        }                                                                                       \
    }
    for (int r0 = 0; r0 < tm; r0 += TMAX) {
        const int* so = slot_of + r0;
        const int tr = tm - r0 < TMAX ? tm - r0 : TMAX;
        if constexpr (TMAX == 1) EVAMX_RUN(1)
        else if constexpr (TMAX == 2) {
            if (tr <= 1) EVAMX_RUN(1)
            else EVAMX_RUN(2)
        } else if constexpr (TMAX == 4) {
            if (tr <= 2) EVAMX_RUN(2)
            else EVAMX_RUN(4)
        } else {
            static_assert(TMAX == 8, "row bounds are 1, 2, 4 or 8");
            if (tr <= 1) EVAMX_RUN(1)
            else if (tr <= 2) EVAMX_RUN(2)
            else if (tr <= 4) EVAMX_RUN(4)
            else EVAMX_RUN(8)
        }
    }
#undef EVAMX_RUN
}

// Runtime rate (k2 = 2K) -> instantiated GEMV; integer rates 2..5.
template <int TMAX>
__device__ __forceinline__ void gemv_dispatch_k(int k2, const uint32_t* trellis, int nt_n, int cg, int c0, int c1,
                                                const GlobalRows& src, const int* slot_of, int tm, float* part,
                                                size_t part_stride)
{
    switch (k2) {
        case 4: gemv_chunk<2, TMAX>(trellis, nt_n, cg, c0, c1, src, slot_of, tm, part, part_stride); break;
        case 6: gemv_chunk<3, TMAX>(trellis, nt_n, cg, c0, c1, src, slot_of, tm, part, part_stride); break;
        case 8: gemv_chunk<4, TMAX>(trellis, nt_n, cg, c0, c1, src, slot_of, tm, part, part_stride); break;
        case 10: gemv_chunk<5, TMAX>(trellis, nt_n, cg, c0, c1, src, slot_of, tm, part, part_stride); break;
        default: break;
    }
}

// Smallest compiled row bound that covers `rows` rows per chunk (wider chunks loop over it).
inline int tmax_for(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

// Sum over the wave of one value per lane (order fixed by the butterfly).
__device__ __forceinline__ float wave_sum(float v)
{
    const int lane = threadIdx.x & 63;
    v += xor_lane_f<1>(v, lane);
    v += xor_lane_f<2>(v, lane);
    v += xor_lane_f<4>(v, lane);
    v += xor_lane_f<8>(v, lane);
    v += xor_lane_f<16>(v, lane);
    v += xor_lane_f<32>(v, lane);
    return v;
}

}  // namespace evamx
