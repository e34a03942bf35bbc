// Wave-level decode GEMV and Hadamard helpers shared by the MoE and the single-linear kernels.
//
// GEMV lane layout (wave64): lane = 8*i + q streams tile (kt, 8*cg + i) words q*K..q*K+K-1 with
// one vector load per k-slice and owns output columns 16i+q and 16i+q+8 of the 128-column group
// for all 16 k of the tile, so the k-loop needs no cross-lane reduction and a wave's 128 columns
// are exactly one Hadamard chunk. The 16 decoded k of a column pair up as (k, k+1). The MoE
// decode path multiplies them on the matrix cores (gemv_wave_m4: each lane quad is one
// v_mfma_f32_4x4x4_16b_f16 block); the single linear's GEMV meets the activation pairs
// (x[2m], x[2m+1]) in v_dot2_f32_f16 (gemv_wave), both with fp32 accumulation.
#pragma once
#include "evamx_device.hpp"

#include <type_traits>

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

// The same transform for a chunk held as consecutive pairs, element e = 2*lane + h: stage 0 is
// in-lane, stages 1..6 pair lanes xor 1..32. Same stage order and operand pairs as had128_lane,
// so the results are bit-identical.
__device__ __forceinline__ void had128_pair(float& v0, float& v1, int lane)
{
    {
        const float a = v0, c = v1;
        v0 = a + c;
        v1 = a - c;
    }
    v0 = bfly_x<1>(v0, lane);  v1 = bfly_x<1>(v1, lane);
    v0 = bfly_x<2>(v0, lane);  v1 = bfly_x<2>(v1, lane);
    v0 = bfly_x<4>(v0, lane);  v1 = bfly_x<4>(v1, lane);
    v0 = bfly_x<8>(v0, lane);  v1 = bfly_x<8>(v1, lane);
    v0 = bfly_x<16>(v0, lane); v1 = bfly_x<16>(v1, lane);
    v0 = bfly_x<32>(v0, lane); v1 = bfly_x<32>(v1, lane);
    v0 *= R_SCALE;
    v1 *= R_SCALE;
}

// The codebook's affine map applied to a column's sums: sum_k x_k w_k = 0x1eee * sum_k x_k h_k +
// 0xc931 * sum_k x_k, with one explicit fused multiply-add, so that no kernel's row count can change
// how the compiler contracts it (a row's bits must not depend on its call's row count).
__device__ __forceinline__ float mul1_affine(float acc, float xs)
{
    return __builtin_fmaf(MUL1_K_INV, acc, MUL1_K_BIAS * xs);
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

// A lane's words of one k-slice: its K words with one non-temporal 64/96/128-bit buffer load
// (+1 dword at K=5), and the word before them in the tile's circular bit string (the last word
// of the previous lane of the tile, or the tile's last word for the first lane) with one more
// dword load from the same cache lines. Buffer loads take the wave-uniform slice offset in a
// scalar register and the per-lane offsets as constant vector offsets, so a step spends no
// vector instructions on addresses.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int BUF_NT = 2;                          // cache policy: non-temporal
constexpr int BUF_WORD3 = 0x00020000;              // raw 32-bit buffer resource on gfx9-family parts

// Resource of a wave-uniform base (the pointer is made provably uniform, so the descriptor lives
// in scalar registers and no load needs a per-lane loop over descriptors).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const uint32_t* base)
{
    const uint64_t v = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    uint32_t* u = (uint32_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, 0x7fffffff, BUF_WORD3);
}

template <int K>
__device__ __forceinline__ void load_slice(LaneWords<K>& w, __amdgpu_buffer_rsrc_t rsrc, uint32_t soff,
                                           uint32_t lane_off, uint32_t prev_off)
{
    if constexpr (K == 2) {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, lane_off, soff, BUF_NT));
        w.b[1] = v.x; w.b[2] = v.y;
    } else if constexpr (K == 3) {
        const u32x3 v = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rsrc, lane_off, soff, BUF_NT));
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z;
    } else {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_off, soff, BUF_NT));
        w.b[1] = v.x; w.b[2] = v.y; w.b[3] = v.z; w.b[4] = v.w;
#pragma unroll
        for (int i = 4; i < K; ++i) w.b[i + 1] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, lane_off + 4 * i, soff, BUF_NT);
    }
    w.b[0] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, prev_off, soff, BUF_NT);
}

// ---------------------------------------------------------------------------------------------
// Waves sharing a SIMD issue oldest-first, so without help the oldest races ahead, the youngest
// finishes last, and the SIMD's last stretch runs one wave that cannot hide its own load
// latency. A streaming loop sets its wave's priority from its progress (done of n steps): 3
// below half, 2 to 3/4, 1 to 9/10, then 0, so a wave that is ahead yields to the ones behind
// and the SIMD's waves reach each mark together; only the last tenth is issued oldest-first.
__device__ __forceinline__ void progress_priority(int done, int n)
{
    if (10 * done >= 9 * n) __builtin_amdgcn_s_setprio(0);
    else if (4 * done >= 3 * n) __builtin_amdgcn_s_setprio(1);
    else if (2 * done >= n) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(3);
}

// ---------------------------------------------------------------------------------------------
// Rate geometry and per-slice decode of the lane layout (lane = 8*i + q owns tile i's columns q
// and q + 8 for the 16 k of a k-slice), shared by the decode GEMV and the MFMA path.

// K2 = 2 x bits: even for integer rates (K = K2/2 words per lane), odd for rates b + 0.5.
template <int K2>
struct Rate {
    static constexpr bool HALF = (K2 & 1) != 0;
    static constexpr int B = K2 / 2;                          // whole bits (half rates)
    static constexpr int K = HALF ? B + 1 : K2 / 2;           // words loaded per lane besides b[0]
    static constexpr int TW = HALF ? 4 * (2 * B + 1) : 8 * K; // words per tile
};

// Byte offsets of a lane's words within its tile (lane_off: the K words, prev_off: the word
// before them in the tile's circular bit string) and, at half rates, the normalising shift.
template <int K2>
__device__ __forceinline__ void lane_offsets(int lane, uint32_t& lane_off, uint32_t& prev_off, uint32_t& sh)
{
    using R = Rate<K2>;
    const int q = lane & 7;
    sh = 0;
    if constexpr (!R::HALF) {
        lane_off = 4u * (uint32_t)((lane >> 3) * R::TW + q * R::K);
        prev_off = 4u * (uint32_t)((lane >> 3) * R::TW + (q == 0 ? R::TW - 1 : q * R::K - 1));
    } else {
        // words s0 .. s0+B+1 cover the lane's bits and the 16 before them; s0 = -1 (q = 0) wraps
        // to the tile's last word, which is loaded on its own like the integer rates' b[0]
        const int r0 = 16 * q * (2 * R::B + 1);
        const int s0 = (r0 - 17 + 32) / 32 - 1;              // floor((r0 - 17) / 32)
        lane_off = 4u * (uint32_t)((lane >> 3) * R::TW + s0 + 1);
        prev_off = 4u * (uint32_t)((lane >> 3) * R::TW + (q == 0 ? R::TW - 1 : s0));
        sh = (q & 1) ? 0u : 16u;
    }
}

// The (1024 + bytesum) pairs of the lane's 32 positions of one k-slice:
// wp[4u + 2c + kh] = column q + 8c, k = 8kh + 2u and 8kh + 2u + 1 (low half: even k).
template <int K2>
__device__ __forceinline__ void decode_slice(const LaneWords<Rate<K2>::K>& w, uint32_t sh, half2_t (&wp)[16])
{
    using R = Rate<K2>;
    constexpr int K = R::K, B = R::B;
    if constexpr (!R::HALF) {
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
    } else {
        uint32_t N[B + 1];
#pragma unroll
        for (int k = 0; k <= B; ++k) N[k] = __builtin_amdgcn_alignbit(w.b[k], w.b[k + 1], sh);
#define EVAMX_DEC_UNIT(U)                                \
        wp[4 * U + 0] = half_hpair<B, 8 * U + 0>(N);     \
        wp[4 * U + 1] = half_hpair<B, 8 * U + 2>(N);     \
        wp[4 * U + 2] = half_hpair<B, 8 * U + 4>(N);     \
        wp[4 * U + 3] = half_hpair<B, 8 * U + 6>(N);
        EVAMX_DEC_UNIT(0)
        EVAMX_DEC_UNIT(1)
        EVAMX_DEC_UNIT(2)
        EVAMX_DEC_UNIT(3)
#undef EVAMX_DEC_UNIT
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

// Activation source of gemv_wave: the 8 fp16 pairs (x[16kt + 2i], x[16kt + 2i + 1]) of row m
// at k-slice kt. XScalar reads rows of global memory through wave-uniform addresses (scalar
// loads into SGPRs); XLds reads rows the wave staged in LDS itself (one uniform-address
// ds_read_b128 pair, a broadcast).
template <int TM>
struct XScalar {
    const half2_t* A;
    uint32_t aoff[TM];      // row m starts at A + 4 * aoff[m] (aoff in 16-byte units)
    __device__ __forceinline__ void load(int m, int kt, half2_t (&d)[8]) const
    {
        const half2_t* xp = A + ((size_t)aoff[m] * 4 + (size_t)kt * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = xp[i];
    }
};

// The rows are written and read as uint32_t words (one type, so that no alias rule separates
// the wave's stores from its loads); rows and slices are 32-byte aligned, so the eight words of
// a slice merge into wide LDS reads.
struct XLds {
    const uint32_t* base;   // LDS: row m at base + m * row_words, k-slice kt at word 8 * (kt - kt0)
    int row_words;
    int kt0;
    __device__ __forceinline__ void load(int m, int kt, half2_t (&d)[8]) const
    {
        const uint32_t* xp = (const uint32_t*)__builtin_assume_aligned(base + m * row_words + 8 * (kt - kt0), 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = __builtin_bit_cast(half2_t, xp[i]);
    }
};

// Orders a wave's LDS writes before its later LDS reads of other lanes' data (and its reads
// before later overwrites): LDS instructions of one wave execute in order, the fence keeps the
// compiler from moving them across.
__device__ __forceinline__ void wave_lds_fence()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Work gemv_wave does around issuing its weight prefetch: issue() runs before the first weight
// loads (loads issued there return first: vector memory loads return in order), finish() once
// they are in flight.
struct NoPrologue {
    static constexpr bool kWork = false;
    __device__ __forceinline__ void issue() {}
    __device__ __forceinline__ void finish() {}
};

// ---------------------------------------------------------------------------------------------
// Decode GEMV over one wave's k-range [kt0, kt1): acc[m][h] += sum_k X[m][k] * h_k,
// h_k = 1024 + bytesum of the weight at (k, col(lane, h)) (see mul1_hpair). The caller zeroes
// acc. `prologue.issue()` runs just before the weight prefetch ring is issued and
// `prologue.finish()` once it is in flight (the rotated-input path loads its activation words
// first and stages its rows in LDS behind the latency of the first weight loads).

// Weight prefetch depth (k-slices in flight per wave). Four slices (4 KiB per wave at 4 bpw)
// measured best for every chunk width once the waves of a SIMD progress together (depths 4..10
// at 1 and 2 rows: 4 and 5 the fastest, 10 4% slower).
template <int TM>
constexpr int prefetch_depth() { return 4; }

template <int K2, int TM, int PF = prefetch_depth<TM>(), typename XS, typename Pro>
__device__ __forceinline__ void gemv_wave(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                          const XS& xs, int tm, float (&acc)[TM][2], Pro& prologue)
{
    using R = Rate<K2>;
    constexpr int K = R::K;
    constexpr int TW = R::TW;
    const int lane = threadIdx.x & 63;
    // the k-range is wave-uniform: keep it (and all index math below) in scalar registers
    kt0 = __builtin_amdgcn_readfirstlane(kt0);
    kt1 = __builtin_amdgcn_readfirstlane(kt1);
    // byte offsets: slices are nt_n tiles apart, the wave's 8 tiles start at tile 8*cg; a
    // projection is at most 7168 x 7168 x 8 bits, far below the 2 GiB buffer range
    const uint32_t slice = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(nt_n * TW));
    const uint32_t cbase = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(cg * 8 * TW));
    const __amdgpu_buffer_rsrc_t rsrc = weight_rsrc(trellis);
    uint32_t lane_off, prev_off, sh;
    lane_offsets<K2>(lane, lane_off, prev_off, sh);

    // Prefetch ring: the row PF slices ahead, clamped to the wave's last row so that the steady
    // state needs no branch and never reads outside the matrix (the clamped reloads hit cache).
    prologue.issue();
    LaneWords<K> ring[PF];
    const int last = kt1 - 1;
#pragma unroll
    for (int d = 0; d < PF; ++d) load_slice<K>(ring[d], rsrc, cbase + (uint32_t)min(kt0 + d, last) * slice, lane_off, prev_off);
    // keep the prologue's work (and its waits for its own loads) after the ring is issued
    if constexpr (Pro::kWork) __builtin_amdgcn_sched_barrier(0);
    prologue.finish();

    // Narrow chunks load the next slice's activations one step ahead, so their latency hides
    // behind a decode instead of stalling every step.
    constexpr bool XPF = TM <= 2;
    half2_t xa[TM][8];
    auto load_x = [&](half2_t (&dst)[TM][8], int kt) {
#pragma unroll
        for (int m = 0; m < TM; ++m)
            if (m < tm) xs.load(m, kt, dst[m]);
    };
    if constexpr (XPF) load_x(xa, kt0);

    // Decode the slot, then refill the same registers with the slice PF ahead (issuing the load
    // before the decode would keep two copies of the slot live and make the compiler rotate
    // registers through moves that wait for every load in flight), then the dot products.
    auto step = [&](int kt, LaneWords<K>& w) {
        half2_t xn[TM][8];
        if constexpr (XPF) load_x(xn, min(kt + 1, last));
        half2_t wp[16];
        decode_slice<K2>(w, sh, wp);
        load_slice<K>(w, rsrc, cbase + (uint32_t)min(kt + PF, last) * slice, lane_off, prev_off);
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m < tm) {
                if constexpr (!XPF) xs.load(m, kt, xa[m]);
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
        // keep the next step's activation loads out of this one (register pressure)
        __builtin_amdgcn_sched_barrier(0);
    };

    const int n_kt = kt1 - kt0;
    int kt = kt0;
    for (; kt + PF <= kt1; kt += PF) {
        progress_priority(kt - kt0, n_kt);
#pragma unroll
        for (int d = 0; d < PF; ++d) step(kt + d, ring[d]);
    }
    progress_priority(n_kt, n_kt);
#pragma unroll
    for (int d = 0; d < PF - 1; ++d)
        if (kt + d < kt1) step(kt + d, ring[d]);
}

// ---------------------------------------------------------------------------------------------
// The same decode GEMV with the products on the matrix cores: v_mfma_f32_4x4x4_16b_f16 runs 16
// independent 4x4x4 blocks, block b on lanes 4b..4b+3, and the decode layout's lane quads are
// exactly such blocks (the four lanes of a quad own four columns of one tile at the same k).
// Lane 4b + j supplies column j of its block as the B operand (the four k of a k-group from its
// decoded pairs) and row j of the block's A operand (the activations of row 4g + j of its 4-row
// group at those k); the block's D holds the four rows of the lane's column in four registers.
// One MFMA thus takes the products of 4 rows x 4 k per lane where v_dot2 takes 1 row x 2 k:
// a k-slice costs 8 MFMAs per 4-row group instead of 16 v_dot2 per row. Rows of a group past the
// call's rows read a copy of the group's first row (their outputs are dropped); a row's result
// does not depend on the other rows of its group.

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x4v_t __attribute__((ext_vector_type(4)));

// Activation rows of the MFMA-product GEMV, staged in LDS: row m at base + m * row_words (a
// padded stride, so that the four rows a lane quad reads sit in different banks), k-slice kt at
// word 8 * (kt - kt0). Lane l reads row 4g + (l & 3) of group g.
template <int NG>
struct XLds4 {
    const uint32_t* base;
    int off[NG];            // this lane's row offset (words) in each group
    int kt0;
    __device__ __forceinline__ void init(const uint32_t* b, int row_words, int k0, int tm)
    {
        base = b;
        kt0 = k0;
        const int j = threadIdx.x & 3;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int m = 4 * g + j;
            off[g] = (m < tm ? m : 4 * g < tm ? 4 * g : 0) * row_words;
        }
    }
    __device__ __forceinline__ void load(int g, int kt, uint32_t (&d)[8]) const
    {
        const uint32_t* xp = (const uint32_t*)__builtin_assume_aligned(base + off[g] + 8 * (kt - kt0), 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = xp[i];
    }
};

// B operand of one MFMA: column c (0: q, 1: q + 8) of the lane, k-group kg (k = 4 kg .. 4 kg + 3)
// of the slice's decoded pairs (wp[4u + 2c + kh] holds k = 8 kh + 2u, 8 kh + 2u + 1).
__device__ __forceinline__ half4_t m4_b(const half2_t (&wp)[16], int c, int kg)
{
    const int kh = kg >> 1, u = 2 * (kg & 1);
    const half2_t lo = wp[4 * u + 2 * c + kh], hi = wp[4 * (u + 1) + 2 * c + kh];
    return half4_t{lo.x, lo.y, hi.x, hi.y};
}

__device__ __forceinline__ half4_t m4_a(const uint32_t (&a)[8], int kg)
{
    const half2_t lo = __builtin_bit_cast(half2_t, a[2 * kg]), hi = __builtin_bit_cast(half2_t, a[2 * kg + 1]);
    return half4_t{lo.x, lo.y, hi.x, hi.y};
}

// acc[g][c][i] += sum_k X[4g + i][k] * h_k over the wave's k-range [kt0, kt1) for the lane's column
// c, for tm >= 1 rows; groups g with 4g >= tm are skipped. Same ring, decode and prologue protocol
// as gemv_wave.
template <int K2, int NG, int PF = 4, typename Pro>
__device__ __forceinline__ void gemv_wave_m4(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                             const XLds4<NG>& xs, int tm, f32x4v_t (&acc)[NG][2], Pro& prologue)
{
    using R = Rate<K2>;
    constexpr int K = R::K;
    constexpr int TW = R::TW;
    const int lane = threadIdx.x & 63;
    kt0 = __builtin_amdgcn_readfirstlane(kt0);
    kt1 = __builtin_amdgcn_readfirstlane(kt1);
    const uint32_t slice = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(nt_n * TW));
    const uint32_t cbase = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(cg * 8 * TW));
    const __amdgpu_buffer_rsrc_t rsrc = weight_rsrc(trellis);
    uint32_t lane_off, prev_off, sh;
    lane_offsets<K2>(lane, lane_off, prev_off, sh);

    prologue.issue();
    LaneWords<K> ring[PF];
    const int last = kt1 - 1;
#pragma unroll
    for (int d = 0; d < PF; ++d) load_slice<K>(ring[d], rsrc, cbase + (uint32_t)min(kt0 + d, last) * slice, lane_off, prev_off);
    if constexpr (Pro::kWork) __builtin_amdgcn_sched_barrier(0);
    prologue.finish();

    // The loop over the k-slices for NA active groups (the groups holding rows), with no branch
    // inside a step: a per-group test in the step splits it into blocks that serialise the
    // decode and the products.
    auto run = [&](auto na) {
        constexpr int NA = decltype(na)::value;
        // a step reads its slice's activations from LDS first: the decode hides their latency
        auto step = [&](int kt, LaneWords<K>& w) {
            uint32_t xa[NA][8];
#pragma unroll
            for (int g = 0; g < NA; ++g) xs.load(g, kt, xa[g]);
            half2_t wp[16];
            decode_slice<K2>(w, sh, wp);
            load_slice<K>(w, rsrc, cbase + (uint32_t)min(kt + PF, last) * slice, lane_off, prev_off);
#pragma unroll
            for (int kg = 0; kg < 4; ++kg)
#pragma unroll
                for (int g = 0; g < NA; ++g) {
                    const half4_t a = m4_a(xa[g], kg);
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        acc[g][c] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, m4_b(wp, c, kg), acc[g][c], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
        };

        const int n_kt = kt1 - kt0;
        int kt = kt0;
        for (; kt + PF <= kt1; kt += PF) {
            progress_priority(kt - kt0, n_kt);
#pragma unroll
            for (int d = 0; d < PF; ++d) step(kt + d, ring[d]);
        }
        progress_priority(n_kt, n_kt);
#pragma unroll
        for (int d = 0; d < PF - 1; ++d)
            if (kt + d < kt1) step(kt + d, ring[d]);
    };
    static_assert(NG == 1 || NG == 2 || NG == 4, "decode path row groups: 1, 2 or 4");
    if constexpr (NG == 1) {
        run(std::integral_constant<int, 1>{});
    } else if constexpr (NG == 2) {
        if (tm > 4) run(std::integral_constant<int, 2>{});
        else run(std::integral_constant<int, 1>{});
    } else {
        // four groups: 9 to 16 rows (9-12 rows too: the fourth group's products are dropped)
        run(std::integral_constant<int, 4>{});
    }
}

// sum of sp[c0], sp[c0 + d], ... below c1, added in that order from 0 (as a sequential loop
// does), the loads of up to B terms issued before their adds: one memory round trip per B terms
// instead of one per term (a loop that adds each load before issuing the next waits a full round
// trip per term).
template <int B>
__device__ __forceinline__ float strided_sum(const float* sp, int c0, int c1, int d = 1)
{
    float xs = 0.0f;
    for (int c = c0; c < c1; c += B * d) {
        float t[B];
#pragma unroll
        for (int j = 0; j < B; ++j) t[j] = gptr<float>(sp)[c + j * d < c1 ? c + j * d : c];
#pragma unroll
        for (int j = 0; j < B; ++j)
            if (c + j * d < c1) xs += t[j];
    }
    return xs;
}

// GEMV for a chunk of tm rows over the 128-element k-chunks [c0, c1) with the smallest
// template that fits; writes fp32 partials part[slot_of[m] * part_stride + column] =
// sum_k x_k w_k = 0x1eee * sum_k x_k h_k + 0xc931 * sum_k x_k.
// Only the row variants up to TMAX are compiled in, so a launch for narrow chunks is not
// register-allocated for the widest one. A chunk of more than TMAX rows (possible only when
// given routes repeat an expert within a token) is processed TMAX rows at a time.
template <int K2, int TMAX>
__device__ __forceinline__ void gemv_chunk(const uint32_t* trellis, int nt_n, int cg, int c0, int c1,
                                           const GlobalRows& src, const int* slot_of, int tm, float* part,
                                           size_t part_stride)
{
    const int lane = threadIdx.x & 63;
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#define EVAMX_RUN(TMV)                                                                          \
    {                                                                                           \
        XScalar<TMV> xsrc;                                                                      \
        xsrc.A = (const half2_t*)src.A;                                                         \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m)                                         \
            xsrc.aoff[m] = (uint32_t)__builtin_amdgcn_readfirstlane((m < tr ? so[m] : so[0]) *   \
                                                                    (int)(src.stride / 8));     \
        float acc[TMV][2];                                                                      \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m) acc[m][0] = acc[m][1] = 0.0f;           \
        NoPrologue none;                                                                        \
        gemv_wave<K2, TMV>(trellis, nt_n, cg, 8 * c0, 8 * c1, xsrc, tr, acc, none);              \
        _Pragma("unroll") for (int m = 0; m < TMV; ++m) {                                       \
            if (m < tr) {                                                                       \
                const int row = so[m];                                                          \
                const float xs = strided_sum<4>(src.sums + (size_t)row * src.sums_stride, c0, c1); \
                float* dst = part + (size_t)row * part_stride;                                  \
                dst[col0] = mul1_affine(acc[m][0], xs);                                         \
                dst[col1] = mul1_affine(acc[m][1], xs);                                         \
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

// Smallest compiled row bound that covers `rows` rows per chunk (wider chunks loop over it).
inline int tmax_for(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

// Sum over the wave of one value per lane (order fixed by the butterfly).
__device__ __forceinline__ float wave_sum(float v)
{
    const int lane = threadIdx.x & 63;
    v = pair_sum<1>(v, lane);
    v = pair_sum<2>(v, lane);
    v = pair_sum<4>(v, lane);
    v = pair_sum<8>(v, lane);
    v = pair_sum<16>(v, lane);
    v = pair_sum<32>(v, lane);
    return v;
}

}  // namespace evamx
