// Device-side building blocks for the EXL3 MoE path on gfx950 (wave64).
//
// Trellis format and codebook: runtime/ds41/csrc/moe_coop3072/vendor/quant/exl3_dq.cuh:15-31
// (bit windows), codebook.cuh:86-99 (MUL1 decode). Hadamard evaluation order:
// hadamard_inner.cuh:17-44 and exl3_moe_coop_kernel.cuh:131-147.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace evamx {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;

// Rates (k2 = 2 x bits) the decode GEMV is instantiated for: 1.5 .. 4 in steps of 0.5, and 5.
__host__ __device__ constexpr bool gemv_k2_supported(int k2) { return (k2 >= 3 && k2 <= 8) || k2 == 10; }
constexpr float R_SCALE = 0.088388347648f;   // 1/sqrt(128) as the reference spells it

__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, int s)
{
    // ((hi:lo) >> s) low 32 bits; s is a compile-time constant at every call site (v_alignbit)
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> s);
}

// MUL1 hash of a 16-bit state sitting in the low (HI=false) or high (HI=true) half of r:
// state * 0x83DCD12D mod 2^32, split as state*0xD12D + ((state*0x83DC) mod 2^16) << 16 so that
// it maps to a 16-bit multiply with a word-1 destination (SDWA) and a 16x16->32 multiply-add,
// instead of the multi-pass 32-bit multiply.
// Written in inline asm: the compiler otherwise folds the split back into v_mul_lo_u32, or
// masks the half with an extra instruction instead of using the 16-bit operand selects.
template <bool HI>
__device__ __forceinline__ uint32_t mul1_hash(uint32_t r)
{
    uint32_t y, p;
    if constexpr (HI) {
        asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD"
            : "=v"(y) : "v"(r), "v"(0x83DCu));
        asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(p) : "v"(r), "v"(0xD12Du), "v"(y));
    } else {
        asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:DWORD"
            : "=v"(y) : "v"(r), "v"(0x83DCu));
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(p) : "v"(r), "v"(0xD12Du), "v"(y));
    }
    return p;
}

// Two decoded weights (fp16, bit-exact MUL1 decode) from two hashes:
// h = fp16_bits(0x6400 + bytesum) = 1024 + bytesum, w = fma_fp16(h, 0x1eee, 0xc931).
__device__ __forceinline__ half2_t mul1_pair(uint32_t p0, uint32_t p1)
{
    uint32_t s = __builtin_amdgcn_sad_u8(p0, 0u, 0x64006400u);
    s = __builtin_amdgcn_sad_hi_u8(p1, 0u, s);
    const half2_t h = __builtin_bit_cast(half2_t, s);
    const half2_t k = {__builtin_bit_cast(half_t, (uint16_t)0x1eee), __builtin_bit_cast(half_t, (uint16_t)0x1eee)};
    const half2_t b = {__builtin_bit_cast(half_t, (uint16_t)0xc931), __builtin_bit_cast(half_t, (uint16_t)0xc931)};
    return __builtin_elementwise_fma(h, k, b);
}

// The fp16 pair (1024 + bytesum) of two hashes, before the codebook's affine map: the decode
// GEMV multiplies these by the activations and applies w = 0x1eee * h + 0xc931 once per column
// (sum_k x_k w_k = 0x1eee * sum_k x_k h_k + 0xc931 * sum_k x_k).
__device__ __forceinline__ half2_t mul1_hpair(uint32_t p0, uint32_t p1)
{
    uint32_t s = __builtin_amdgcn_sad_u8(p0, 0u, 0x64006400u);
    s = __builtin_amdgcn_sad_hi_u8(p1, 0u, s);
    return __builtin_bit_cast(half2_t, s);
}

constexpr float MUL1_K_INV = 0.00676727294921875f;   // fp16 0x1eee
constexpr float MUL1_K_BIAS = -10.3828125f;          // fp16 0xc931

__device__ __forceinline__ half_t mul1_one(uint32_t state)
{
    const half2_t w = mul1_pair(mul1_hash<false>(state), 0u);
    return w.x;
}

__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c)
{
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

// ---------------------------------------------------------------------------------------------
// Lane-local window geometry.
//
// A lane owns 32 consecutive positions of a 16x16 tile: the positions of reference lanes
// 4q..4q+3 (q = lane % 8), i.e. columns q and q+8 for all 16 k of the tile. For an integer
// rate K those positions end inside the lane's K words, and the first windows reach back
// into the previous word (the last word of lane q-1 of the same tile, circularly). The bit
// string B = prev:W0:...:W(K-1) (MSB first) holds position j's window at bits
// [E(j)-16, E(j)) with E(j) = 32 + (j+1)K.

template <int K>
struct LaneWords {
    uint32_t b[K + 1];   // b[0] = previous word of the tile's bit string, b[1..K] = own words
};

template <int K>
__device__ __forceinline__ constexpr int win_end(int j) { return 32 + (j + 1) * K; }

// Register whose low 16 bits are the window ending at E (and whose high 16 bits are the
// window ending at E-16).
template <int K, int E>
__device__ __forceinline__ uint32_t win_reg(const LaneWords<K>& w)
{
    constexpr int L = (E - 1) / 32;
    constexpr int S = 32 * (L + 1) - E;
    static_assert(L >= 1 && L <= K, "window outside the lane's words");
    return funnel(w.b[L - 1], w.b[L], S);
}

// Hash of lane-local position j (0..31). When K divides 16, the windows of positions j and
// j + 16/K are 16 bits apart and share one funnel shift: with P = 16/K, positions in odd
// P-blocks take the low half of their own register, positions in even P-blocks the high half
// of the register of j + P.
template <int K, int J>
__device__ __forceinline__ uint32_t lane_hash(const LaneWords<K>& w)
{
    constexpr int E = win_end<K>(J);
    if constexpr (16 % K == 0) {
        constexpr int P = 16 / K;
        if constexpr ((J / P) % 2 == 0)
            return mul1_hash<true>(win_reg<K, E + 16>(w));
        else
            return mul1_hash<false>(win_reg<K, E>(w));
    } else {
        return mul1_hash<false>(win_reg<K, E>(w));
    }
}

// Decoded weight pair of lane-local positions (J, J+1) (J even): same column, k and k+1.
template <int K, int J>
__device__ __forceinline__ half2_t lane_pair(const LaneWords<K>& w)
{
    return mul1_pair(lane_hash<K, J>(w), lane_hash<K, J + 1>(w));
}

// The (1024 + bytesum) pair of the same positions (see mul1_hpair).
template <int K, int J>
__device__ __forceinline__ half2_t lane_hpair(const LaneWords<K>& w)
{
    return mul1_hpair(lane_hash<K, J>(w), lane_hash<K, J + 1>(w));
}

// ---------------------------------------------------------------------------------------------
// Half-integer rates b + 0.5 (exl3_dq.cuh:254-285): positions alternate b and b+1 bits, odd
// positions carrying the extra bit. A lane's 32 positions then start 16*q*(2b+1) bits into the
// tile, which is word-aligned for even q and half a word off for odd q. The lane normalises its
// words into N[0..b] = the bit string from 16 bits before its first position (one v_alignbit
// each, by 16 or 0 per lane), after which every window sits at a compile-time offset: position
// j ends at bit 16 + (j odd ? (j+1)/2 * (2b+1) : j/2 * (2b+1) + b) of N.

template <int B>
constexpr int half_win_end(int j)
{
    return 16 + ((j & 1) ? ((j + 1) / 2) * (2 * B + 1) : (j / 2) * (2 * B + 1) + B);
}

template <int B, int J>
__device__ __forceinline__ uint32_t half_hash(const uint32_t (&N)[B + 1])
{
    constexpr int E = half_win_end<B>(J);
    constexpr int L = (E - 1) / 32;
    constexpr int S = 32 * (L + 1) - E;
    static_assert(L <= B, "window outside the normalised words");
    return mul1_hash<false>(funnel(N[L > 0 ? L - 1 : 0], N[L], S));
}

template <int B, int J>
__device__ __forceinline__ half2_t half_hpair(const uint32_t (&N)[B + 1])
{
    return mul1_hpair(half_hash<B, J>(N), half_hash<B, J + 1>(N));
}

// ---------------------------------------------------------------------------------------------
// Wave-level 128-point Hadamard in the reference's fp32 evaluation order: radix-2 on element
// bits 0..6 in increasing order, lower index a+b, upper a-b, scale last. Bit-identical to the
// reference for any data layout, because IEEE addition is commutative and each stage's
// operand pairs are the same.

// Value of lane (lane ^ M) for a compile-time M, on the vector ALU only: DPP for M < 16 (quad
// permutes, row rotations) and gfx950's row swaps for 16 and 32. permlane16_swap(v, v) gives
// (rows 0,0,2,2 ; rows 1,1,3,3) of v, so lane ^ 16 reads the first for odd rows and the second
// for even rows; permlane32_swap(v, v) gives (rows 0,1,0,1 ; rows 2,3,2,3) likewise.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int lane)
{
    if constexpr (M == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
    else if constexpr (M == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, false); // quad_perm [2,3,0,1]
    else if constexpr (M == 4) {
        const uint32_t r4 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xf, 0xf, false);       // row_ror:4
        const uint32_t r12 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x12C, 0xf, 0xf, false);      // row_ror:12
        return (lane & 4) ? r4 : r12;
    } else if constexpr (M == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false); // row_ror:8
    else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        static_assert(M == 32, "lane xor 1, 2, 4, 8, 16 or 32");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}

template <int M>
__device__ __forceinline__ float xor_lane_f(float v, int lane)
{
    return __builtin_bit_cast(float, xor_lane<M>(__builtin_bit_cast(uint32_t, v), lane));
}

// The value of the lane that DPP pattern CTRL selects, as an operand the compiler folds into the
// add that consumes it (every lane of the patterns used here has a source, so the bound control
// changes nothing).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// The row swaps of xor_lane<16> and <32> as a pair (A, B): in the lower block of each pair of
// blocks (lane & M clear) A is the lane's own value and B its partner's, in the upper block A is
// the partner's and B its own.
template <int M>
__device__ __forceinline__ void swap_pair(float v, float& a, float& b)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        a = __builtin_bit_cast(float, (uint32_t)r[0]);
        b = __builtin_bit_cast(float, (uint32_t)r[1]);
    } else {
        static_assert(M == 32, "row swaps: lane xor 16 or 32");
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        a = __builtin_bit_cast(float, (uint32_t)r[0]);
        b = __builtin_bit_cast(float, (uint32_t)r[1]);
    }
}

// Butterfly where the partner p lives in lane ^ M; the upper lane (stage bit set) takes a - b:
// v + p in the lower lane, p - v in the upper one, computed as p + (+-v) (the same IEEE sums: a
// sign flip is exact) so that the DPP lane read folds into the add; for M = 16, 32 as A + (+-B)
// from the row swap's pair, which is v + p in the lower block and p - v in the upper one.
template <int M>
__device__ __forceinline__ float bfly_x(float v, int lane)
{
    if constexpr (M == 16 || M == 32) {
        float a, b;
        swap_pair<M>(v, a, b);
        return a + ((lane & M) ? -b : b);
    } else {
        const float sv = (lane & M) ? -v : v;
        if constexpr (M == 4) {
            // both rotations in every lane, then a select: a DPP read inside a lane-dependent
            // branch would run with half the lanes off and read them as zeros
            const float r4 = dpp_f<0x124>(v) + sv, r12 = dpp_f<0x12C>(v) + sv;             // row_ror:4 / :12
            return (lane & 4) ? r4 : r12;
        } else if constexpr (M == 8) {
            return dpp_f<0x128>(v) + sv;                                                     // row_ror:8
        } else {
            return dpp_f<M == 1 ? 0xB1 : 0x4E>(v) + sv;                                      // quad_perm
        }
    }
}

// v + (v of lane ^ M) in every lane, the lane read folded into the add as in bfly_x.
template <int M>
__device__ __forceinline__ float pair_sum(float v, int lane)
{
    if constexpr (M == 16 || M == 32) {
        float a, b;
        swap_pair<M>(v, a, b);
        return a + b;
    } else if constexpr (M == 4) {
        const float r4 = dpp_f<0x124>(v) + v, r12 = dpp_f<0x12C>(v) + v;                   // as in bfly_x
        return (lane & 4) ? r4 : r12;
    } else if constexpr (M == 8) {
        return dpp_f<0x128>(v) + v;
    } else {
        return dpp_f<M == 1 ? 0xB1 : 0x4E>(v) + v;
    }
}

// ---------------------------------------------------------------------------------------------
// Results that cross workgroups inside one launch: the producers store them write-through
// (relaxed device-scope atomic stores, which go to the memory side), wait for the stores'
// acknowledgements and arrive at a counter; the last to arrive reads them from the memory side
// (sc1 loads), so neither side needs a cache-wide fence.

__device__ __forceinline__ void store_wt(float* d, float v)
{
    __hip_atomic_store(d, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int LD_SC1 = 16;            // buffer load cache policy: device scope (sc1)

// Arrival counter: one 64-bit word, high half a tag, low half the arrivals. A word at rest holds
// (ARRIVE_REST, 0); each of the n arrivals adds 1 and the one whose add brings the count to n is
// the last, which puts the word back to rest for the next call (graph replays included), so a
// call needs no clearing launch. A word in any other state (a workspace's first use: its bytes
// are whatever the memory held) is detected by the add's old value; such an arrival's add is not
// counted, and it counts itself with compare-and-swap instead, adding 1 to a counting word (an
// (ARRIVE_FIX, c) word, or an (ARRIVE_REST, c) word that the garbage's adds carried into) or
// taking any other word to (ARRIVE_FIX, 1); later adds onto a counting word count as usual. Each
// arrival is counted exactly once either way (tests/test_arrive_protocol.py runs the protocol over
// random interleavings and initial words), and the swap loop ends since each failed swap means
// another arrival succeeded. The tags have four distinct bytes, so fill patterns of one repeated
// byte never pass for a counting word. Device-scope adds on one word cost about 12 ns each when
// they queue (504 workgroups on one word: 7.4 us against 1.7 us spread out), nothing measurable
// at a few tens per word.
constexpr unsigned ARRIVE_REST = 0x3c6ef372u;
constexpr unsigned ARRIVE_FIX = 0xa54ff53au;
// Counters sit a cache line (128 bytes) apart.
constexpr int ARRIVE_STRIDE = 16;

__device__ __forceinline__ bool arrive_counting(unsigned long long w, unsigned n)
{
    const unsigned hi = (unsigned)(w >> 32);
    return (hi == ARRIVE_REST || hi == ARRIVE_FIX) && (unsigned)w < n;
}

__device__ __forceinline__ bool arrive_last(unsigned long long* word, unsigned n)
{
    const unsigned long long old = __hip_atomic_fetch_add(word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool last;
    if (arrive_counting(old, n)) {
        last = (unsigned)old + 1 == n;
    } else {
        unsigned long long cur = old + 1;       // refreshed by the first failed swap
        for (;;) {
            // a counting word (of either tag) counts the arrivals made since it became one: add
            // this one; anything else (garbage) restarts the count at this arrival
            const unsigned long long next = arrive_counting(cur, n) ? cur + 1 : ((unsigned long long)ARRIVE_FIX << 32) | 1ull;
            if (__hip_atomic_compare_exchange_strong(word, &cur, next, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)) {
                last = (unsigned)next == n;
                break;
            }
        }
    }
    if (last) __hip_atomic_store(word, (unsigned long long)ARRIVE_REST << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return last;
}

// A wave's arrival once its write-through stores are acknowledged: true in every lane of the
// last of n arrivals (lane 0 adds).
__device__ __forceinline__ bool wave_arrive_last(unsigned long long* word, unsigned n)
{
    __builtin_amdgcn_s_waitcnt(0);
    int l = 0;
    if ((threadIdx.x & 63) == 0) l = arrive_last(word, n);
    return __builtin_amdgcn_readfirstlane(l) != 0;
}

}  // namespace evamx
