// Device helpers of the decode-shaped MoE pipeline, shared by its kernels: portable router
// scores and top-k, grouping, input rotations, expert pointers (moe_prepare.hip,
// moe_gate_up*.hip, moe_down.hip, moe_epilogue.hip; the launch sequence is in moe_decode.hip).
#pragma once
#include <cstdlib>
#include <cstring>
#include "evamx_gemv.hpp"
#include "evamx_internal.hpp"
#include "evamx_moe.hpp"

namespace evamx {

// ---------------------------------------------------------------------------------------------
// Portable fp32 score functions (mul/add only, contraction off) so that router scores agree bit
// for bit with the CPU restatement.

#pragma clang fp contract(off)
// exp by Cody-Waite range reduction (x = n ln2 + r, ln2 split in a 16-bit head and a tail so
// that n * head is exact) and the degree-7 Taylor polynomial of e^r on |r| <= ln2/2.
inline __device__ float exp_portable(float x)
{
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float n = rintf(x * 1.4426950408889634f);
    const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187e-06f;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)n);
}

inline __device__ float log1p_portable(float u)
{
    const float s = u / (2.0f + u);
    const float s2 = s * s;
    float p = 1.0f / 15.0f;
    p = p * s2 + 1.0f / 13.0f;
    p = p * s2 + 1.0f / 11.0f;
    p = p * s2 + 1.0f / 9.0f;
    p = p * s2 + 1.0f / 7.0f;
    p = p * s2 + 1.0f / 5.0f;
    p = p * s2 + 1.0f / 3.0f;
    p = p * s2 + 1.0f;
    return 2.0f * (s * p);
}

inline __device__ float score_fn(float z, int fn)
{
    if (fn == EVAMX_SCORE_SIGMOID) return 1.0f / (1.0f + exp_portable(-z));
    const float sp = fmaxf(z, 0.0f) + log1p_portable(exp_portable(-fabsf(z)));
    return sqrtf(sp);
}

inline __device__ float route_weight(float s, float tot, float scale)
{
    const float w = s / (tot + 1e-20f);
    return w * scale;
}
#pragma clang fp contract(on)

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// bf16 <-> fp32 with round-to-nearest-even (finite values; NaN stays NaN)
__device__ __forceinline__ float bf16_value(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t bf16_bits(float f)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}


// ---------------------------------------------------------------------------------------------
// Router front: logits[r][e] = sum_k float(x[r][k]) * gate_w[e][k] in fp32 (Block.route's
// x.float() @ gate_w.T, model.py:404-409). One wave per (expert, group of GATE_ROWS rows): lane l
// takes k = 4l + 256j (one float4 of the weight row per step, reused by the group's rows) with a
// sequential fma chain, and the lanes' partials meet in a fixed butterfly, so a row's logits
// depend on that row alone whatever the batch (the per-row stable_linear of model.py:158-165).

constexpr int GATE_ROWS = 8;

// x as the fp16 value the reference routes and runs the experts on: Block.experts casts the
// activations to fp16 first (model.py:455), so a bf16 x is rounded to fp16 (values beyond the
// fp16 range become inf, the fp16 subnormal range keeps fp16 precision).
__device__ __forceinline__ float x_fp16_value(uint16_t b, int dtype)
{
    if (dtype == EVAMX_DTYPE_F16) return h2f(__builtin_bit_cast(half_t, b));
    return h2f(f2h(__builtin_bit_cast(float, (uint32_t)b << 16)));
}

__device__ __forceinline__ float x_at(const MoeParams& p, int r, int k)
{
    return x_fp16_value(((const uint16_t*)p.x)[(size_t)r * p.x_stride + k], p.x_dtype);
}

// ---------------------------------------------------------------------------------------------
// Router keys are packed as (order-preserving key bits << 32 | ~index) so that one 64-bit max, reduced
// with lane butterflies, yields the winner and the tie rule at once (+0 and -0 compare equal).

__device__ __forceinline__ uint64_t pack_key(float k, int e)
{
    if (k == 0.0f) k = 0.0f;
    const uint32_t u = __builtin_bit_cast(uint32_t, k);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

// Maximum of one 32-bit value per lane over the wave, in every lane: quad maxima by two quad
// permutations, row maxima by rotations of 4 and 8 within the row, then across rows.
// The DPP reads are operands the compiler folds into the max (every lane of these patterns has a
// source); across rows, the row swap's pair holds the lane's own value and its partner's in some
// order, so their max is the pair's.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v, int lane)
{
    (void)lane;
    v = max(v, dpp_u<0xB1>(v));                          // quad_perm [1,0,3,2]
    v = max(v, dpp_u<0x4E>(v));                          // quad_perm [2,3,0,1]
    v = max(v, dpp_u<0x124>(v));                         // row_ror:4
    v = max(v, dpp_u<0x128>(v));                         // row_ror:8
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)r16[0], (uint32_t)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = max((uint32_t)r32[0], (uint32_t)r32[1]);
    return v;
}

// The lane holding the wave's largest key (one head key per lane): the largest high word, and
// among lanes tied on it the largest low word (the lowest expert index).
__device__ __forceinline__ int wave_argmax_key(uint64_t k, int lane)
{
    const uint32_t hk = (uint32_t)(k >> 32);
    const uint32_t m = __builtin_amdgcn_readfirstlane(wave_max_u32(hk, lane));
    const uint64_t tie = __ballot(hk == m);
    if (__builtin_amdgcn_readfirstlane(__popcll(tie)) == 1) return __ffsll((long long)tie) - 1;
    const uint32_t lo = hk == m ? (uint32_t)k : 0u;
    const uint32_t ml = __builtin_amdgcn_readfirstlane(wave_max_u32(lo, lane));
    return __ffsll((long long)__ballot(hk == m && (uint32_t)k == ml)) - 1;
}

// Compare-exchange of two (key, logit) entries into descending key order.
__device__ __forceinline__ void ce_desc(uint64_t& ka, float& za, uint64_t& kb, float& zb)
{
    const bool sw = kb > ka;
    const uint64_t k = sw ? kb : ka;
    kb = sw ? ka : kb;
    ka = k;
    const float z = sw ? zb : za;
    zb = sw ? za : zb;
    za = z;
}

// Top-k of row r: lane j < topk ends with winner j's expert index and routing weight.
template <int NPER>
__device__ __forceinline__ void route_winners(const MoeParams& p, int r, int lane, int& id, float& w)
{
    static_assert(NPER == 4 || NPER == 8, "4 or 8 keys per lane");
    const float* z = p.logits + (size_t)r * p.n_logits;
    float zr[NPER];
    uint64_t key[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        zr[i] = e < p.n_logits ? z[e] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        float k = -INFINITY;
        if (e < p.n_logits) {
            const float zz = zr[i];
            if (p.sel_bias) k = score_fn(zz, p.score) + p.sel_bias[e];
            else k = (p.score == EVAMX_SCORE_SIGMOID) ? zz : score_fn(zz, p.score);
        }
        key[i] = e < p.n_logits ? pack_key(k, e) : 0ull;
    }
    // each lane sorts its keys (descending; Batcher networks, checked by the zero-one principle),
    // so a round's candidate of a lane is its head and the winner's lane just pops it
    if constexpr (NPER == 4) {
        ce_desc(key[0], zr[0], key[1], zr[1]); ce_desc(key[2], zr[2], key[3], zr[3]);
        ce_desc(key[0], zr[0], key[2], zr[2]); ce_desc(key[1], zr[1], key[3], zr[3]);
        ce_desc(key[1], zr[1], key[2], zr[2]);
    } else {
        constexpr int net[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                                    {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
        for (int c = 0; c < 19; ++c) ce_desc(key[net[c][0]], zr[net[c][0]], key[net[c][1]], zr[net[c][1]]);
    }
    // winners one at a time; lane j keeps winner j's index and logit
    float my_z = 0.0f;
    int my_id = 0;
    for (int j = 0; j < p.topk; ++j) {
        const int wl = __builtin_amdgcn_readfirstlane(wave_argmax_key(key[0], lane));
        const int bi = (int)(0xffffffffu - (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], wl));
        const float zb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, zr[0]), wl));
        if (lane == wl) {
#pragma unroll
            for (int i = 0; i + 1 < NPER; ++i) {
                key[i] = key[i + 1];
                zr[i] = zr[i + 1];
            }
            key[NPER - 1] = 0ull;
        }
        if (lane == j) { my_z = zb; my_id = bi; }
    }
    // scores of the winners in parallel, their total in slot order
    const float sc = lane < p.topk ? score_fn(my_z, p.score) : 0.0f;
    float tot = 0.0f;
    for (int j = 0; j < p.topk; ++j)
        tot = tot + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), j));
    id = my_id;
    w = lane < p.topk ? route_weight(sc, tot, p.route_scale) : 0.0f;
}

template <int NPER>
inline __device__ void route_token_n(const MoeParams& p, int r, int lane, int* sel_o, half_t* rw_o, bool publish)
{
    int my_id;
    float w;
    route_winners<NPER>(p, r, lane, my_id, w);
    if (lane < p.topk) {
        const int s = r * p.topk + lane;
        if (sel_o) sel_o[s] = my_id;
        if (rw_o) rw_o[s] = f2h(w);
        if (publish) {
            p.sel[s] = my_id;
            p.weights[s] = w;
            p.rw16[s] = f2h(w);
        }
    }
}

// Routing of one token by one wave: top-k by (key desc, index asc); weights from the scores.
// Lane j < topk writes slot j to sel_o / rw_o and, when publishing, to the global outputs.
__device__ __forceinline__ void route_token(const MoeParams& p, int r, int lane, int* sel_o, half_t* rw_o, bool publish)
{
    if (p.n_logits <= 256) route_token_n<4>(p, r, lane, sel_o, rw_o, publish);
    else route_token_n<EVAMX_MAX_EXPERTS / 64>(p, r, lane, sel_o, rw_o, publish);
}

__device__ __forceinline__ void route_lanes(const MoeParams& p, int r, int lane, int& id, float& w)
{
    if (p.n_logits <= 256) route_winners<4>(p, r, lane, id, w);
    else route_winners<EVAMX_MAX_EXPERTS / 64>(p, r, lane, id, w);
}

// ---------------------------------------------------------------------------------------------
// Grouping by one workgroup. Per-slot arrays (local, order) may live in LDS or global memory;
// per-expert arrays live in LDS.

struct ExpertLds {
    int cnt[EVAMX_MAX_EXPERTS + 1];
    int off[EVAMX_MAX_EXPERTS + 1];
    int run_base[EVAMX_MAX_EXPERTS + 1];
    int chunk_base[EVAMX_MAX_EXPERTS + 1];
    int unit_base[EVAMX_MAX_EXPERTS + 1];
    int fill[EVAMX_MAX_EXPERTS];
    int small_base[EVAMX_MAX_EXPERTS + 1];   // MFMA tiles of at most 16 rows (decode path: units of
                                             // experts of more than EVAMX_CHUNK rows)
    int large_base[EVAMX_MAX_EXPERTS + 1];   // MFMA tiles of more than 16 rows (decode path: units
                                             // of experts of 5 to EVAMX_CHUNK rows)
};

// Decode path: the first unit of expert e when units are numbered longest first (experts of more
// than EVAMX_CHUNK rows, then of 5 to EVAMX_CHUNK rows, then the rest; expert order within each),
// so that the GEMV launches start their longest waves first.
__device__ __forceinline__ int unit_order_base(const ExpertLds& ex, int E, int e)
{
    const int n = ex.cnt[e];
    if (n > EVAMX_CHUNK) return ex.small_base[e];
    if (n > 4) return ex.small_base[E] + ex.large_base[e];
    return ex.small_base[E] + ex.large_base[E] + (ex.unit_base[e] - ex.small_base[e] - ex.large_base[e]);
}

// Work units (summed chunk weights) of an expert with n active slots.
__device__ __forceinline__ int expert_units(const MoeParams& p, int n)
{
    const int full = n / EVAMX_CHUNK, rest = n % EVAMX_CHUNK;
    return full * unit_mult(p, EVAMX_CHUNK) + (rest ? unit_mult(p, rest) : 0);
}

// Inclusive scan over the wave of one int per lane, on the vector ALU: row-local DPP shifts
// (row_shr 1, 2, 4, 8, zero fill), then the row totals carried forward (row_bcast:15 into
// rows 1 and 3, row_bcast:31 into rows 2 and 3).
__device__ __forceinline__ int wave_incl_scan(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
    return v;
}

// Per-expert offsets by one wave, from the slot counts cnt[0..E): exclusive prefix sums of the
// counts (off), of the 8-slot runs (run_base), of the chunks of chunk_rows_of(p) slots
// (chunk_base), of the GEMV work units (unit_base) and, for the MFMA path, of the tiles of at most
// and of more than 16 rows (small_base, large_base), each with its total at [E]. Lane l owns
// experts PER*l .. PER*l + PER-1 in registers; the six lane-total scans run together.
template <int PER>
inline __device__ void expert_offsets(const MoeParams& p, ExpertLds& ex, int lane)
{
    const int E = p.n_local;
    const int cs = 31 - __builtin_clz(chunk_rows_of(p));      // chunk rows are a power of two
    const int e0 = lane * PER;
    int v[6][PER], tot[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int n = e0 + i < E ? ex.cnt[e0 + i] : 0;
        v[0][i] = n;
        v[1][i] = (n + 7) >> 3;
        v[2][i] = (n + (1 << cs) - 1) >> cs;
        v[3][i] = p.mfma ? v[2][i] : expert_units(p, n);          // MFMA tiles are one unit each
        // MFMA tiles by size: at most 16 rows (small) or more (large); with tiles of at most 16
        // rows every tile is small, with 64-row tiles the full ones and a remainder of more
        // than 16 rows are large
        // Decode path: the units of experts of more than EVAMX_CHUNK rows and of 5 to EVAMX_CHUNK
        // rows (the strict prepare numbers units longest first, unit_order_base).
        const int rest = n & ((1 << cs) - 1);
        if (p.mfma) {
            v[4][i] = cs <= 4 ? v[2][i] : (rest > 0 && rest <= 16 ? 1 : 0);
            v[5][i] = cs <= 4 ? 0 : (n >> cs) + (rest > 16 ? 1 : 0);
        } else {
            v[4][i] = n > EVAMX_CHUNK ? v[3][i] : 0;
            v[5][i] = n > 4 && n <= EVAMX_CHUNK ? v[3][i] : 0;
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) tot[k] += v[k][i];
    }
    int run[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) run[k] = wave_incl_scan(tot[k]);
    int* const dst[6] = {ex.off, ex.run_base, ex.chunk_base, ex.unit_base, ex.small_base, ex.large_base};
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        int r = run[k] - tot[k];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if (e0 + i < E) dst[k][e0 + i] = r;
            r += v[k][i];
        }
        if (lane == 63) dst[k][E] = run[k];
    }
}

// Activity of one slot (exl3_moe_coop_kernel.cuh:208-223): its local expert, or -1 when its fp16
// weight is zero, its expert is outside [min_expert, max_expert), or the local index is out of
// bounds (which also sets the sticky flag when flag is set).
__device__ __forceinline__ int slot_local(const MoeParams& p, int64_t e, half_t rw, bool flag)
{
    if (h2f(rw) == 0.0f) return -1;
    int64_t le = e;
    if (p.min_expert >= 0) {
        if (!(e >= p.min_expert && e < p.max_expert)) return -1;
        le = e - p.min_expert;
    }
    if (le < 0 || le >= p.n_local) {
        if (flag) atomicOr(p.err, EVAMX_ERR_EXPERT_RANGE);
        return -1;
    }
    return (int)le;
}

// Slot activity (exl3_moe_coop_kernel.cuh:208-223) -> local[s] = local expert or -1 (bounds
// violations set the sticky flag and make the slot inactive), then the stable order of the
// active slots by (expert, slot) and, when publishing, the reference run table.
template <typename SelT>
inline __device__ void group_slots(const MoeParams& p, const SelT* sel, const half_t* rw, int slots, int* local,
                            int* order, ExpertLds& ex, bool publish)
{
    const int t = threadIdx.x, nt = blockDim.x, lane = t & 63, wave = t >> 6;
    const int E = p.n_local;
    for (int e = t; e < E; e += nt) { ex.cnt[e] = 0; ex.fill[e] = 0; }
    __syncthreads();
    for (int s = t; s < slots; s += nt) {
        const int lo = slot_local(p, (int64_t)sel[s], rw[s], publish);
        local[s] = lo;
        if (lo >= 0) atomicAdd(&ex.cnt[lo], 1);
    }
    __syncthreads();
    if (wave == 0) {
        if (E <= 256) expert_offsets<4>(p, ex, lane);
        else expert_offsets<EVAMX_MAX_EXPERTS / 64>(p, ex, lane);
        // Stable scatter by (expert, slot): blocks of 64 slots in order; lanes holding the same
        // expert find each other with one ballot per expert-index bit.
        for (int s0 = 0; s0 < slots; s0 += 64) {
            const int s = s0 + lane;
            const int e = s < slots ? local[s] : -1;
            const bool act = e >= 0;
            uint64_t m = __ballot(act);
#pragma unroll
            for (int b = 0; b < 10; ++b) {
                const bool bit = act && ((e >> b) & 1);
                const uint64_t bb = __ballot(bit);
                m &= bit ? bb : ~bb;
            }
            const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            int rank = 0;
            if (act) {
                rank = ex.fill[e] + __popcll(m & lt);
                const int pos = ex.off[e] + rank;
                if (order) order[pos] = s;
                if (publish && p.runs) {
                    p.runs[2 + p.slots_max + 1 + pos] = s;
                    if ((rank & 7) == 0) p.runs[2 + ex.run_base[e] + rank / 8] = pos;
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (act && (m & lt) == 0) ex.fill[e] += __popcll(m);
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
}

// The same grouping for many slots by a workgroup of GROUP_WAVES waves: wave w owns the
// contiguous slot range [w*per, (w+1)*per); per-wave expert histograms give every wave the
// offsets of its first slot of each expert, so all waves scatter at once and the order stays
// stable by (expert, slot). local/order live in global memory.
constexpr int GROUP_WAVES = 16;

struct GroupLds {
    int hist[GROUP_WAVES][EVAMX_MAX_EXPERTS];
};

template <typename SelT>
inline __device__ void group_slots_par(const MoeParams& p, const SelT* sel, const half_t* rw, int slots, int* local,
                                int* order, ExpertLds& ex, GroupLds& gl, bool publish)
{
    const int t = threadIdx.x, nt = blockDim.x, lane = t & 63, wave = t >> 6;
    const int E = p.n_local;
    for (int i = t; i < GROUP_WAVES * EVAMX_MAX_EXPERTS; i += nt) (&gl.hist[0][0])[i] = 0;
    __syncthreads();
    const int per = (slots + GROUP_WAVES - 1) / GROUP_WAVES;
    const int s0 = wave * per, s1 = min(slots, s0 + per);
    for (int s = s0 + lane; s < s1; s += 64) {
        const int64_t e = (int64_t)sel[s];
        const float w = h2f(rw[s]);
        int lo = -1;
        if (w != 0.0f) {
            int64_t le = e;
            bool ok = true;
            if (p.min_expert >= 0) {
                ok = e >= p.min_expert && e < p.max_expert;
                le = e - p.min_expert;
            }
            if (ok) {
                if (le < 0 || le >= E) {
                    if (publish) atomicOr(p.err, EVAMX_ERR_EXPERT_RANGE);
                } else lo = (int)le;
            }
        }
        local[s] = lo;
        if (lo >= 0) atomicAdd(&gl.hist[wave][lo], 1);
    }
    __syncthreads();
    // per-wave exclusive offsets within each expert (in place) and the expert totals
    for (int e = t; e < E; e += nt) {
        int run = 0;
#pragma unroll
        for (int w = 0; w < GROUP_WAVES; ++w) {
            const int c = gl.hist[w][e];
            gl.hist[w][e] = run;
            run += c;
        }
        ex.cnt[e] = run;
    }
    __syncthreads();
    if (wave == 0) {
        if (E <= 256) expert_offsets<4>(p, ex, lane);
        else expert_offsets<EVAMX_MAX_EXPERTS / 64>(p, ex, lane);
    }
    __syncthreads();
    for (int b = s0; b < s1; b += 64) {
        const int s = b + lane;
        const int e = s < s1 ? local[s] : -1;      // this lane's own store above
        const bool act = e >= 0;
        uint64_t m = __ballot(act);
#pragma unroll
        for (int bit = 0; bit < 10; ++bit) {
            const bool v = act && ((e >> bit) & 1);
            const uint64_t bb = __ballot(v);
            m &= v ? bb : ~bb;
        }
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        if (act) {
            const int rank = gl.hist[wave][e] + __popcll(m & lt);
            const int pos = ex.off[e] + rank;
            if (order) order[pos] = s;
            if (publish && p.runs) {
                p.runs[2 + p.slots_max + 1 + pos] = s;
                if ((rank & 7) == 0) p.runs[2 + ex.run_base[e] + rank / 8] = pos;
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (act && (m & lt) == 0) gl.hist[wave][e] += __popcll(m);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
}

// Chunks of <= chunk_rows_of(p) slots per expert, then the shared expert's rows; for the decode
// GEMV also their work units (unit -> chunk map) and each slot's chunk weight. `order` is the
// grouped slot order.
// MFMA mode: files tile ci under its size class, in chunk (expert) order within each class: the
// tiles of at most 16 rows from the front of p.tiles, the larger ones from the back. si / li
// are the tile's index within its class (with 64-row tiles an expert has at most one small
// tile, its last; with 16-row tiles all of its tiles are small).
__device__ __forceinline__ void file_tile(const MoeParams& p, int ci, int rows, int si, int li)
{
    if (rows <= 16) p.tiles[si] = ci;
    else p.tiles[p.max_chunks - 1 - li] = ci;
}

inline __device__ void write_chunks(const MoeParams& p, const ExpertLds& ex, const int* order)
{
    const int t = threadIdx.x, nt = blockDim.x;
    const int E = p.n_local;
    const int CR = chunk_rows_of(p);
    const int n_active = ex.off[E];
    for (int e = t; e < E; e += nt) {
        const int n = ex.cnt[e];
        int u = ex.unit_base[e];
        for (int j = 0; j * CR < n; ++j) {
            const int ci = ex.chunk_base[e] + j;
            const int rows = min(CR, n - j * CR);
            const int m = p.mfma ? 1 : unit_mult(p, rows);
            int* c = p.chunks + 8 * ci;
            c[0] = e;
            c[1] = ex.off[e] + j * CR;
            c[2] = rows;
            c[3] = k2_gu_of(p, e);
            c[6] = k2_d_of(p, e);
            if ((!gemv_k2_supported(c[3]) || !gemv_k2_supported(c[6])) && j == 0) atomicOr(p.err, EVAMX_ERR_RATE);
            c[4] = u;
            c[5] = m;
            c[7] = 0;
            for (int i = 0; i < m; ++i) p.unit_chunk[u + i] = ci;
            if (!p.mfma)                 // MFMA tiles weigh 1: filled in parallel below
                for (int i = 0; i < rows; ++i) p.slot_mult[order[c[1] + i]] = m;
            else
                file_tile(p, ci, rows, ex.small_base[e] + (CR <= 16 ? j : 0), ex.large_base[e] + j);
            u += m;
        }
    }
    if (p.has_shared) {
        const int base = ex.chunk_base[E];
        const int nsc = (p.T + CR - 1) / CR;
        const int slots = p.T * p.topk;
        for (int j = t; j < nsc; j += nt) {
            const int rows = min(CR, p.T - j * CR);
            const int m = p.mfma ? 1 : unit_mult(p, rows);
            const int u = ex.unit_base[E] + j * (p.mfma ? 1 : unit_mult(p, CR));     // earlier chunks are full
            int* c = p.chunks + 8 * (base + j);
            c[0] = -1;
            c[1] = n_active + j * CR;
            c[2] = rows;
            c[3] = p.k2_shared;
            c[4] = u;
            c[5] = m;
            c[6] = p.k2_shared_d;
            c[7] = 0;
            for (int i = 0; i < m; ++i) p.unit_chunk[u + i] = base + j;
            if (!p.mfma)
                for (int i = 0; i < rows; ++i) p.slot_mult[slots + j * CR + i] = m;
            else                         // shared tiles follow the routed ones
                file_tile(p, base + j, rows, ex.small_base[E] + (CR <= 16 ? j : 0), ex.large_base[E] + j);
        }
    }
    if (p.mfma) {
        for (int s = t; s < moe_nslot(p); s += nt) p.slot_mult[s] = 1;
        if (t == 0) {
            const int sh_rest = p.has_shared ? p.T % CR : 0;
            const int sh_tiles = p.has_shared ? (p.T + CR - 1) / CR : 0;
            p.meta[3] = ex.small_base[E] + (CR <= 16 ? sh_tiles : (sh_rest > 0 && sh_rest <= 16 ? 1 : 0));
        }
    }
}

__device__ __forceinline__ int total_chunks(const MoeParams& p, const ExpertLds& ex)
{
    return ex.chunk_base[p.n_local] + (p.has_shared ? (p.T + chunk_rows_of(p) - 1) / chunk_rows_of(p) : 0);
}

__device__ __forceinline__ int total_units(const MoeParams& p, const ExpertLds& ex)
{
    const int CR = chunk_rows_of(p);
    return ex.unit_base[p.n_local] + (p.has_shared ? (p.mfma ? (p.T + CR - 1) / CR : expert_units(p, p.T)) : 0);
}

// ---------------------------------------------------------------------------------------------
// Input rotations fp16(H128(x * suh)) of the grouped rows, with their 128-chunk sums. Work is
// cut into units (grouped row o, gate|up) of H/128 chunks, and each unit into `parts` equal
// chunk ranges so that the waves of the grid have one range each (grid-stride beyond that).
// A wave resolves its row's slot, expert and suh pointer once, then works through its chunks
// in batches whose x and suh loads are all issued before the first butterfly.

constexpr int ROT_BATCH = 8;

__device__ __forceinline__ float x_elem(uint32_t w, int hi, int dtype)
{
    return x_fp16_value((uint16_t)(hi ? w >> 16 : w), dtype);
}

// A wave-uniform 64-bit value through two 32-bit readfirstlanes (the builtin takes an int).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Chunks [c0, c1) of grouped slot s (routed slot < T*topk with local expert e, or shared row).
inline __device__ void rotate_chunks(const MoeParams& p, int s, int e, int proj, int c0, int c1, int lane)
{
    const int slots = p.T * p.topk;
    const bool shared = s >= slots;
    const int row = shared ? s - slots : s / p.topk;
    const int trow = proj == 0 ? EVAMX_TBL_G_SUH : EVAMX_TBL_U_SUH;
    // the shared pointer selected by value: a select of addresses into the kernel argument (an
    // indexed access) puts the whole argument in scratch memory
    const uint64_t sg = uniform_u64((uint64_t)p.sh_ptr[EVAMX_TBL_G_SUH]);
    const uint64_t su = uniform_u64((uint64_t)p.sh_ptr[EVAMX_TBL_U_SUH]);
    const half_t* suh = shared ? (const half_t*)(proj == 0 ? sg : su)
                               : (const half_t*)p.tables[(size_t)trow * p.tbl_stride + e];
    const uint32_t* xw = (const uint32_t*)((const uint16_t*)p.x + (size_t)row * p.x_stride) + lane;
    const uint32_t* sw = (const uint32_t*)suh + lane;
    uint32_t* dst = (uint32_t*)(p.xr + ((size_t)proj * p.nslot_max + s) * p.H) + lane;
    float* sums = p.xsum + ((size_t)proj * p.nslot_max + s) * (p.H / 128);
    for (int b = c0; b < c1; b += ROT_BATCH) {
        uint32_t xv[ROT_BATCH], sv[ROT_BATCH];
#pragma unroll
        for (int j = 0; j < ROT_BATCH; ++j) {
            if (b + j < c1) {
                xv[j] = xw[(b + j) * 64];
                sv[j] = sw[(b + j) * 64];
            }
        }
#pragma unroll
        for (int j = 0; j < ROT_BATCH; ++j) {
            if (b + j < c1) {
                const half2_t su = __builtin_bit_cast(half2_t, sv[j]);
                float v0 = x_elem(xv[j], 0, p.x_dtype) * h2f(su.x);
                float v1 = x_elem(xv[j], 1, p.x_dtype) * h2f(su.y);
                if (shared) {
                    // shared EXL3 linear: fp16 product (hadamard_inner.cuh:109-115); routed
                    // experts: fp32 product (exl3_moe_coop_kernel.cuh:186-191)
                    v0 = h2f(f2h(x_elem(xv[j], 0, p.x_dtype) * h2f(su.x)));
                    v1 = h2f(f2h(x_elem(xv[j], 1, p.x_dtype) * h2f(su.y)));
                }
                had128_pair(v0, v1, lane);
                const half2_t r = {f2h(v0), f2h(v1)};
                dst[(b + j) * 64] = __builtin_bit_cast(uint32_t, r);
                const float sum = wave_sum(h2f(r.x) + h2f(r.y));
                if (lane == 0) sums[b + j] = sum;
            }
        }
    }
}

// Rotations of n_rows rows by the waves [w0, w0 + nw) of the grid: grouped rows order[0..n_rows),
// or, with order null, slots 0..n_rows (routed slots then shared rows; inactive slots skipped).
inline __device__ void rotate_rows(const MoeParams& p, const int* order, const int* local, int n_rows, int w, int nw, int lane)
{
    const int nch = p.H / 128;
    const int units = n_rows * 2;
    if (units == 0) return;
    int parts = nw / units;
    parts = parts < 1 ? 1 : (parts > nch ? nch : parts);
    const int slots = p.T * p.topk;
    for (int it = w; it < units * parts; it += nw) {
        const int u = it / parts, part = it - u * parts;
        const int o = u >> 1, proj = u & 1;
        const int s = order ? __builtin_amdgcn_readfirstlane(order[o]) : o;
        const int e = s < slots ? __builtin_amdgcn_readfirstlane(local[s]) : -1;
        if (s < slots && e < 0) continue;                 // inactive slot (slot enumeration only)
        rotate_chunks(p, s, e, proj, nch * part / parts, nch * (part + 1) / parts, lane);
    }
}

// ---------------------------------------------------------------------------------------------
// Prepare of the decode path (calls of at most EVAMX_GEMV_MAX_ROWS rows): one workgroup routes,
// groups, publishes the run table and writes the unit and slot records; the input rotations
// happen inside the gate/up GEMV waves, each for its own k-range.

// Bitonic sort of one 32-bit key per lane across the wave, ascending in lane order: stages on
// lane bits (size 2..64, stride size/2..1), each a compare-exchange with lane ^ stride.
template <int SIZE, int STRIDE>
__device__ __forceinline__ uint32_t bitonic_stage(uint32_t k, int lane)
{
    const uint32_t o = xor_lane<STRIDE>(k, lane);
    const bool up = (lane & SIZE) == 0;                 // ascending block (SIZE 64: all lanes)
    const bool lower = (lane & STRIDE) == 0;
    return (lower == up) ? (k < o ? k : o) : (k > o ? k : o);
}

template <int SIZE, int STRIDE>
__device__ __forceinline__ uint32_t bitonic_merge(uint32_t k, int lane)
{
    k = bitonic_stage<SIZE, STRIDE>(k, lane);
    if constexpr (STRIDE > 1) k = bitonic_merge<SIZE, STRIDE / 2>(k, lane);
    return k;
}

__device__ __forceinline__ uint32_t wave_sort_asc(uint32_t k, int lane)
{
    k = bitonic_merge<2, 1>(k, lane);
    k = bitonic_merge<4, 2>(k, lane);
    k = bitonic_merge<8, 4>(k, lane);
    k = bitonic_merge<16, 8>(k, lane);
    k = bitonic_merge<32, 16>(k, lane);
    k = bitonic_merge<64, 32>(k, lane);
    return k;
}

// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ const void* expert_ptr(const MoeParams& p, int e, int row)
{
    if (e < 0) return (const void*)p.sh_ptr[row];
    return (const void*)p.tables[(size_t)row * p.tbl_stride + e];
}

// Slots slot[0..tm) of a unit record (entries past tm repeat slot[0]); the record is not written
// during the GEMV launch, so these are scalar loads.
template <int TM>
__device__ __forceinline__ void record_slots(const int* slot, int tm, int (&so)[TM])
{
    const __attribute__((address_space(4))) int* sl = (const __attribute__((address_space(4))) int*)slot;
#pragma unroll
    for (int m = 0; m < TM; ++m) so[m] = __builtin_amdgcn_readfirstlane(sl[m < tm ? m : 0]);
}

// A slot record through scalar loads (the records are written by an earlier launch and only read
// after it), field by field. (One 16-dword vector load of the whole record failed the decode-path
// parity tests, which pass with these per-field loads; its cause was not found.)
__device__ __forceinline__ SlotRec load_slot_rec(const SlotRec* rp)
{
    const __attribute__((address_space(4))) SlotRec* c = (const __attribute__((address_space(4))) SlotRec*)rp;
    SlotRec r;
    r.active = c->active;
    r.shared = c->shared;
    r.s_gu = c->s_gu;
    r.s_d = c->s_d;
    r.w = c->w;
    r.g_svh = c->g_svh;
    r.u_svh = c->u_svh;
    r.d_suh = c->d_suh;
    r.d_svh = c->d_svh;
    return r;
}

}  // namespace evamx
