// Decode-shaped cooperative EXL3 MoE layer on gfx950.
//
// Replaces the reference's prepare/rot/A/B launch sequence
// (runtime/ds41/csrc/moe_coop3072/moe_coop3072.cu:42-71). Cross-workgroup results only ever
// cross a kernel boundary: a device-scope release fence costs an L2 write-back on this
// multi-XCD part, far more than a launch when thousands of waves would each need one. Five
// stages on one stream, no host synchronisation, no memset (graph-capturable):
//
//   (gate)        optional router front: fp32 logits x . gate_w (model.py:404-409)
//   moe_prepare   routing (optional), slot activity + bounds flag, stable grouping by expert
//                 (the reference run table, runs <= 8 slots: prepare_runs.cuh:8-66; and chunks
//                 of <= 8 slots for the GEMV work items, or tiles of <= 64 for the MFMA path),
//                 then the input rotation fp16(H128(x * suh)) of every active slot
//                 (exl3_moe_coop_kernel.cuh:613-629; shared expert: fp16 pre-scale,
//                 hadamard_inner.cuh:109-115). For 3-16 rows one kernel: every workgroup
//                 routes, workgroup 0 groups and publishes the tables, the others rotate.
//                 Decode path (1-2 rows): unit and slot records instead of tables, no rotation
//                 launch (the gate/up waves rotate their own inputs); 2 rows: one workgroup;
//                 1 row: no prepare launch (the gate/up launch routes).
//   moe_gate_up   per (unit, gate|up, 128 columns, k-split) wave: decode GEMV -> fp32 partials
//                 (3 rows and more: MFMA tiles, moe_prefill.hip)
//   moe_act       per (active slot, 128 columns of I): sums the gate/up partials in fixed
//                 order, rounds to fp16 (gu_f32 = false), and runs the activation epilogue
//                 (exl3_moe_coop_kernel.cuh:758-806; shared expert: model.py:450-452)
//   moe_down      per (chunk, 128 columns, k-split) wave: decode GEMV -> fp32 partials
//                 (3 rows and more: MFMA tiles)
//   moe_combine   per (token, 128 columns): output rotation * svh * routing weight, summed over
//                 the token's slots in slot order, plus the shared expert
//                 (exl3_moe_coop_kernel.cuh:860-962, model.py:498)
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
__device__ float exp_portable(float x)
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

__device__ float log1p_portable(float u)
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

__device__ float score_fn(float z, int fn)
{
    if (fn == EVAMX_SCORE_SIGMOID) return 1.0f / (1.0f + exp_portable(-z));
    const float sp = fmaxf(z, 0.0f) + log1p_portable(exp_portable(-fabsf(z)));
    return sqrtf(sp);
}

__device__ float route_weight(float s, float tot, float scale)
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

__global__ __launch_bounds__(256) void moe_gate_kernel(MoeParams p, float* logits)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    const int ngr = (p.T + GATE_ROWS - 1) / GATE_ROWS;
    if (wid >= p.n_logits * ngr) return;
    const int e = wid / ngr, r0 = (wid - e * ngr) * GATE_ROWS;
    const float4* w = (const float4*)(p.gate_w + (size_t)e * p.H);
    float acc[GATE_ROWS];
#pragma unroll
    for (int r = 0; r < GATE_ROWS; ++r) acc[r] = 0.0f;
    for (int k4 = lane; k4 < p.H / 4; k4 += 64) {
        const float4 wv = w[k4];
#pragma unroll
        for (int r = 0; r < GATE_ROWS; ++r) {
            if (r0 + r < p.T) {
                const int k = 4 * k4;
                float a = acc[r];
                a = fmaf(x_at(p, r0 + r, k + 0), wv.x, a);
                a = fmaf(x_at(p, r0 + r, k + 1), wv.y, a);
                a = fmaf(x_at(p, r0 + r, k + 2), wv.z, a);
                a = fmaf(x_at(p, r0 + r, k + 3), wv.w, a);
                acc[r] = a;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GATE_ROWS; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && r0 + r < p.T) logits[(size_t)(r0 + r) * p.n_logits + e] = v;
    }
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
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v, int lane)
{
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, false));    // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, false));    // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xf, 0xf, false));   // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false));   // row_ror:8
    v = max(v, xor_lane<16>(v, lane));
    v = max(v, xor_lane<32>(v, lane));
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
__device__ void route_token_n(const MoeParams& p, int r, int lane, int* sel_o, half_t* rw_o, bool publish)
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
    int small_base[EVAMX_MAX_EXPERTS + 1];   // MFMA tiles of at most 16 rows
    int large_base[EVAMX_MAX_EXPERTS + 1];   // MFMA tiles of more than 16 rows
};

// Work units (summed chunk weights) of an expert with n active slots.
__device__ __forceinline__ int expert_units(int n)
{
    const int full = n / EVAMX_CHUNK, rest = n % EVAMX_CHUNK;
    return full * chunk_mult(EVAMX_CHUNK) + (rest ? chunk_mult(rest) : 0);
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
__device__ void expert_offsets(const MoeParams& p, ExpertLds& ex, int lane)
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
        v[3][i] = p.mfma ? v[2][i] : expert_units(n);          // MFMA tiles are one unit each
        // MFMA tiles by size: at most 16 rows (small) or more (large); with tiles of at most 16
        // rows every tile is small, with 64-row tiles the full ones and a remainder of more
        // than 16 rows are large
        const int rest = n & ((1 << cs) - 1);
        v[4][i] = !p.mfma ? 0 : cs <= 4 ? v[2][i] : (rest > 0 && rest <= 16 ? 1 : 0);
        v[5][i] = !p.mfma || cs <= 4 ? 0 : (n >> cs) + (rest > 16 ? 1 : 0);
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
__device__ void group_slots(const MoeParams& p, const SelT* sel, const half_t* rw, int slots, int* local,
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
__device__ void group_slots_par(const MoeParams& p, const SelT* sel, const half_t* rw, int slots, int* local,
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

__device__ void write_chunks(const MoeParams& p, const ExpertLds& ex, const int* order)
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
            const int m = p.mfma ? 1 : chunk_mult(rows);
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
            const int m = p.mfma ? 1 : chunk_mult(rows);
            const int u = ex.unit_base[E] + j * (p.mfma ? 1 : chunk_mult(CR));     // earlier chunks are full
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
    return ex.unit_base[p.n_local] + (p.has_shared ? (p.mfma ? (p.T + CR - 1) / CR : expert_units(p.T)) : 0);
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
__device__ void rotate_chunks(const MoeParams& p, int s, int e, int proj, int c0, int c1, int lane)
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
__device__ void rotate_rows(const MoeParams& p, const int* order, const int* local, int n_rows, int w, int nw, int lane)
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
// Prepare for small batches (T*topk <= EVAMX_SMALL_SLOTS, T <= EVAMX_SMALL_ROWS): every
// workgroup routes in LDS, one wave per token (workgroups of max(4, T) waves); workgroup 0
// groups the slots and publishes the tables while the others rotate the active slots' inputs
// (rotations are stored by slot, so they need no order).

constexpr int EVAMX_SMALL_SLOTS = 512;
constexpr int EVAMX_SMALL_ROWS = 16;

struct SmallLds {
    ExpertLds ex;
    int sel[EVAMX_SMALL_SLOTS];
    half_t rw[EVAMX_SMALL_SLOTS];
    int local[EVAMX_SMALL_SLOTS];
    int order[EVAMX_SMALL_SLOTS + EVAMX_SMALL_ROWS];
};

__global__ __launch_bounds__(64 * EVAMX_SMALL_ROWS) void moe_prepare_small_kernel(MoeParams p)
{
    __shared__ SmallLds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nt = blockDim.x, nwv = nt >> 6;
    const int slots = p.T * p.topk;
    const bool pub = blockIdx.x == 0;
    if (p.logits) {
        for (int r = wave; r < p.T; r += nwv) route_token(p, r, lane, sh.sel, sh.rw, pub);
    } else {
        for (int s = t; s < slots; s += nt) {
            const int64_t e = p.sel[s];
            // indices outside the int range are outside any table: keep them out of range
            sh.sel[s] = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
            sh.rw[s] = p.weights ? f2h(p.weights[s]) : p.rw16[s];
            if (pub && p.weights) p.rw16[s] = sh.rw[s];
        }
    }
    if (pub && p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += nt) p.runs[i] = 0;
    }
    __syncthreads();
    if (!pub) {
        // rotation workgroups need only each slot's expert: the grouping is workgroup 0's
        for (int s = t; s < slots; s += nt) sh.local[s] = slot_local(p, sh.sel[s], sh.rw[s], false);
        __syncthreads();
        rotate_rows(p, nullptr, sh.local, slots + (p.has_shared ? p.T : 0), (blockIdx.x - 1) * nwv + wave,
                    (gridDim.x - 1) * nwv, lane);
        return;
    }
    group_slots(p, sh.sel, sh.rw, slots, sh.local, sh.order, sh.ex, pub);
    const int n_active = sh.ex.off[p.n_local];
    if (p.has_shared)
        for (int r = t; r < p.T; r += nt) sh.order[n_active + r] = slots + r;
    __syncthreads();
    {
        for (int s = t; s < slots; s += nt) p.local[s] = sh.local[s];
        for (int i = t; i < n_active + (p.has_shared ? p.T : 0); i += nt) p.order[i] = sh.order[i];
        write_chunks(p, sh.ex, sh.order);
        if (t == 0) {
            p.runs[0] = sh.ex.run_base[p.n_local];
            p.runs[1] = 0;
            p.runs[2 + sh.ex.run_base[p.n_local]] = n_active;
            p.meta[0] = total_chunks(p, sh.ex);
            p.meta[1] = n_active;
            p.meta[2] = total_units(p, sh.ex);
        }
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

// Prepare of the decode path (calls of at most EVAMX_GEMV_MAX_ROWS rows, so at most 64 slots):
// waves [0, T) route one token each while the other waves copy the [9][n_local] pointer table
// (and the per-expert rates) into LDS; then wave 0 alone groups the slots with one key per lane
// sorted across the wave (key (local expert, slot): the stable order by expert), cuts runs of at
// most EVAMX_CHUNK slots at expert changes (the reference run table's runs, which are also the
// GEMV chunks), and writes the run table and the unit and slot records from registers and LDS.
constexpr int GEMV_PREP_WAVES = 4;

struct GemvPrepLds {
    uint64_t tbl[9][EVAMX_MAX_EXPERTS];
    uint8_t k2[EVAMX_MAX_EXPERTS];
    uint8_t k2d[EVAMX_MAX_EXPERTS];
    int sel[64];
    half_t rw[64];
};

__global__ __launch_bounds__(64 * GEMV_PREP_WAVES) void moe_prepare_gemv_kernel(MoeParams p)
{
    __shared__ GemvPrepLds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int slots = p.T * p.topk;               // at most 2 * EVAMX_MAX_TOPK = 64
    const int E = p.n_local;
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += blockDim.x) p.runs[i] = 0;
    }
    if (wave < p.T) {
        if (p.logits) route_token(p, wave, lane, sh.sel, sh.rw, true);      // writes slots wave * topk + j
    } else {
        const int nt = (GEMV_PREP_WAVES - p.T) * 64, i0 = t - p.T * 64;
        for (int i = i0; i < 9 * E; i += nt) sh.tbl[i / E][i % E] = (uint64_t)p.tables[(size_t)(i / E) * p.tbl_stride + i % E];
        for (int i = i0; i < E; i += nt) {
            sh.k2[i] = (uint8_t)k2_gu_of(p, i);
            sh.k2d[i] = (uint8_t)k2_d_of(p, i);
        }
    }
    if (!p.logits && t < slots) {
        const int64_t e = p.sel[t];
        sh.sel[t] = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
        sh.rw[t] = p.weights ? f2h(p.weights[t]) : p.rw16[t];
        if (p.weights) p.rw16[t] = sh.rw[t];
    }
    __syncthreads();
    if (wave != 0) return;

    // slot activity (lane = slot), the published local expert, inactive slot records
    int e = -1;
    if (lane < slots) {
        e = slot_local(p, sh.sel[lane], sh.rw[lane], true);
        p.local[lane] = e;
        if (e < 0) {
            SlotRec q = {};
            p.srec[lane] = q;
        }
    }
    // stable grouping: sort keys (expert, slot); inactive slots sort last
    const uint32_t key = wave_sort_asc(e >= 0 ? ((uint32_t)e << 6) | (uint32_t)lane : 0xffffffffu, lane);
    const bool act = key != 0xffffffffu;
    const int ge = (int)(key >> 6), gs = (int)(key & 63);
    const uint64_t amask = __ballot(act);
    const int n_active = __popcll(amask);
    const int prev_e = __shfl_up(ge, 1, WAVE);
    const uint64_t heads = __ballot(act && (lane == 0 || prev_e != ge));
    const uint64_t le_mask = lane == 63 ? ~0ull : ((2ull << lane) - 1);     // lanes 0..lane
    const int first = 63 - __clzll(heads & le_mask);                        // the expert's first position
    const bool rs = act && ((lane - first) % EVAMX_CHUNK) == 0;             // run (chunk) start
    const uint64_t rmask = __ballot(rs);
    const int n_runs = __popcll(rmask);
    const uint64_t above = rmask & ~le_mask;
    const int next = above ? __ffsll((long long)above) - 1 : n_active;
    const int rows = rs ? next - lane : 0;
    const int m = rs ? chunk_mult(rows) : 0;
    const int m_incl = wave_incl_scan(m);
    const int ubase = m_incl - m;
    const int routed_units = __builtin_amdgcn_readlane(m_incl, 63);
    const KSplit kgu = ks_gate_up(p, p.units_max), kd = ks_down(p, p.units_max);
    // the chunk of each position: its run start's lane
    const int rlane = act ? 63 - __clzll(rmask & le_mask) : 0;
    const int my_m = __shfl(m, rlane, WAVE);
    int slot_run[EVAMX_CHUNK];
#pragma unroll
    for (int j = 0; j < EVAMX_CHUNK; ++j) slot_run[j] = __shfl(gs, lane + j < 64 ? lane + j : 63, WAVE);

    if (act) {
        // run table (moe_coop3072.py:86-106): order, run starts
        if (p.runs) {
            p.runs[2 + p.slots_max + 1 + lane] = gs;
            if (rs) p.runs[2 + __popcll(rmask & (le_mask >> 1)) ] = lane;
        }
        p.order[lane] = gs;
        const int k2 = sh.k2[ge], k2d = sh.k2d[ge];
        SlotRec q;
        q.active = 1;
        q.shared = 0;
        q.s_gu = ks_of_chunk(kgu, my_m);
        q.s_d = ks_of_chunk(kd, my_m);
        q.w = h2f(sh.rw[gs]);
        q.pad[0] = q.pad[1] = q.pad[2] = 0;
        q.g_svh = sh.tbl[EVAMX_TBL_G_SVH][ge];
        q.u_svh = sh.tbl[EVAMX_TBL_U_SVH][ge];
        q.d_suh = sh.tbl[EVAMX_TBL_D_SUH][ge];
        q.d_svh = sh.tbl[EVAMX_TBL_D_SVH][ge];
        p.srec[gs] = q;
        if (rs) {
            if (!gemv_k2_supported(k2) || !gemv_k2_supported(k2d)) atomicOr(p.err, EVAMX_ERR_RATE);
            UnitRec r;
            r.e = ge;
            r.rows = rows;
            r.k2 = k2;
            r.ubase = ubase;
            r.s_gu = ks_of_chunk(kgu, m);
            r.s_d = ks_of_chunk(kd, m);
            r.k2_d = k2d;
            r.pad0 = 0;
#pragma unroll
            for (int j = 0; j < EVAMX_CHUNK; ++j) r.slot[j] = j < rows ? slot_run[j] : slot_run[0];
            r.tr[0] = sh.tbl[EVAMX_TBL_G_TRELLIS][ge];
            r.tr[1] = sh.tbl[EVAMX_TBL_U_TRELLIS][ge];
            r.tr[2] = sh.tbl[EVAMX_TBL_D_TRELLIS][ge];
            r.suh[0] = sh.tbl[EVAMX_TBL_G_SUH][ge];
            r.suh[1] = sh.tbl[EVAMX_TBL_U_SUH][ge];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            for (int i = 0; i < m; ++i) p.urec[ubase + i] = r;
        }
    }
    // the shared expert: one chunk of the T rows after the routed ones
    int n_units = routed_units;
    if (p.has_shared) {
        if (lane < p.T) {
            p.order[n_active + lane] = slots + lane;
            SlotRec q;
            q.active = 1;
            q.shared = 1;
            q.s_gu = ks_of_chunk(kgu, 1);
            q.s_d = ks_of_chunk(kd, 1);
            q.w = 1.0f;
            q.pad[0] = q.pad[1] = q.pad[2] = 0;
            q.g_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SVH];
            q.u_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SVH];
            q.d_suh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SUH];
            q.d_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SVH];
            p.srec[slots + lane] = q;
        }
        if (lane == 0) {
            UnitRec r;
            r.e = -1;
            r.rows = p.T;
            r.k2 = p.k2_shared;
            r.ubase = routed_units;
            r.s_gu = ks_of_chunk(kgu, 1);
            r.s_d = ks_of_chunk(kd, 1);
            r.k2_d = p.k2_shared_d;
            r.pad0 = 0;
#pragma unroll
            for (int j = 0; j < EVAMX_CHUNK; ++j) r.slot[j] = slots + (j < p.T ? j : 0);
            r.tr[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_TRELLIS];
            r.tr[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_TRELLIS];
            r.tr[2] = (uint64_t)p.sh_ptr[EVAMX_TBL_D_TRELLIS];
            r.suh[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SUH];
            r.suh[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SUH];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            p.urec[routed_units] = r;
        }
        n_units += 1;      // T <= 2 rows: one chunk of weight 1
    }
    for (int u = n_units + lane; u < p.units_max; u += 64) p.urec[u].e = EVAMX_NO_UNIT;
    if (lane == 0) {
        if (p.runs) {
            p.runs[0] = n_runs;
            p.runs[1] = 0;
            p.runs[2 + n_runs] = n_active;
        }
        p.meta[0] = n_runs + (p.has_shared ? 1 : 0);
        p.meta[1] = n_active;
        p.meta[2] = n_units;
        p.meta[3] = 0;
    }
}

// ---------------------------------------------------------------------------------------------
// Prepare for any batch, in three launches: routing (one wave per token), grouping (one
// workgroup of 1024 threads, per-slot arrays in global memory), rotations (a full grid).

__global__ __launch_bounds__(256) void moe_route_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int r = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    if (r < p.T) route_token(p, r, lane, nullptr, nullptr, true);
}

__global__ __launch_bounds__(64 * GROUP_WAVES) void moe_group_kernel(MoeParams p)
{
    __shared__ ExpertLds ex;
    __shared__ GroupLds gl;
    const int t = threadIdx.x;
    const int slots = p.T * p.topk;
    if (!p.logits && p.weights)
        for (int s = t; s < slots; s += 1024) p.rw16[s] = f2h(p.weights[s]);
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += 1024) p.runs[i] = 0;
    }
    __syncthreads();
    group_slots_par(p, p.sel, p.rw16, slots, p.local, p.order, ex, gl, true);
    const int n_active = ex.off[p.n_local];
    if (t == 0 && p.runs) {
        p.runs[0] = ex.run_base[p.n_local];
        p.runs[1] = 0;
        p.runs[2 + ex.run_base[p.n_local]] = n_active;
    }
    if (!(p.mode & PREP_MOE)) return;
    if (p.has_shared)
        for (int r = t; r < p.T; r += 1024) p.order[n_active + r] = slots + r;
    __syncthreads();                 // the shared rows of the order are read by write_chunks
    write_chunks(p, ex, p.order);
    if (t == 0) {
        p.meta[0] = total_chunks(p, ex);
        p.meta[1] = n_active;
        p.meta[2] = total_units(p, ex);
    }
}

constexpr int EVAMX_ROTATE_BLOCKS = 2048;

__global__ __launch_bounds__(256) void moe_rotate_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    rotate_rows(p, p.order, p.local, p.meta[1] + (p.has_shared ? p.T : 0), w, gridDim.x * 4, lane);
}

// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ const void* expert_ptr(const MoeParams& p, int e, int row)
{
    if (e < 0) return (const void*)p.sh_ptr[row];
    return (const void*)p.tables[(size_t)row * p.tbl_stride + e];
}

// ---------------------------------------------------------------------------------------------
// Decode path (calls of at most EVAMX_GEMV_MAX_ROWS rows): gate/up waves rotate their own
// inputs. A wave (unit, gate|up, 128 columns, k-split) reads its unit's record, issues its
// weight prefetch, and while the first weight loads are in flight computes fp16(H128(x * suh))
// of its rows over its k-chunks into LDS (with each row's chunk sums, added in chunk order),
// then streams the weights against those LDS rows. The k-range is taken in windows of at most
// ROT_CW chunks (one window at the DSv3 shape).

constexpr int ROT_CW = 16;            // 128-chunks of rotated input per LDS window and row

// Rotations of the tm rows so[0..tm) over the 128-chunks [w0, w1) into LDS (row m at dst + m *
// row_words, chunk w0 + j at word 64 j), adding each chunk's sum to xs[m]: the operations of
// rotate_chunks, so rows and sums are bit-identical to the rotation kernels' output. issue()
// loads the x and suh words of the first ROT_BATCH chunks, finish() rotates and stores them
// (and any further chunks of the window, loading them then).
template <int TM>
struct RotStage {
    static constexpr bool kWork = true;
    const MoeParams& p;
    const int (&so)[TM];
    int tm, w0, w1, row_words, lane;
    __amdgpu_buffer_rsrc_t suh_rsrc, x_rsrc[TM];   // wave-uniform bases: loads take scalar offsets
    uint32_t* dst;
    float (&xs)[TM];
    uint32_t xv[TM][ROT_BATCH], sv[ROT_BATCH];

    __device__ __forceinline__ void load(int b)
    {
        // chunk c of a row is 256 bytes at byte 256 c, lane l's pair at byte 4 l; chunks past the
        // window reload its last one (in bounds, unused), so the loads need no branches
#pragma unroll
        for (int j = 0; j < ROT_BATCH; ++j)
            sv[j] = __builtin_amdgcn_raw_buffer_load_b32(suh_rsrc, 4 * lane, 256 * min(b + j, w1 - 1), 0);
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int j = 0; j < ROT_BATCH; ++j)
                xv[m][j] = __builtin_amdgcn_raw_buffer_load_b32(x_rsrc[m], 4 * lane, 256 * min(b + j, w1 - 1), 0);
    }
    __device__ __forceinline__ void rotate(int b)
    {
        const int slots = p.T * p.topk;
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m >= tm) continue;
            const bool shared = so[m] >= slots;
            uint32_t* d = dst + m * row_words + lane;
#pragma unroll
            for (int j = 0; j < ROT_BATCH; ++j) {
                if (b + j < w1) {
                    const half2_t su = __builtin_bit_cast(half2_t, sv[j]);
                    float v0 = x_elem(xv[m][j], 0, p.x_dtype) * h2f(su.x);
                    float v1 = x_elem(xv[m][j], 1, p.x_dtype) * h2f(su.y);
                    if (shared) {
                        // shared EXL3 linear: fp16 product (hadamard_inner.cuh:109-115)
                        v0 = h2f(f2h(v0));
                        v1 = h2f(f2h(v1));
                    }
                    had128_pair(v0, v1, lane);
                    const half2_t r = {f2h(v0), f2h(v1)};
                    d[(b + j - w0) * 64] = __builtin_bit_cast(uint32_t, r);
                    xs[m] += wave_sum(h2f(r.x) + h2f(r.y));
                }
            }
        }
    }
    __device__ __forceinline__ void issue() { load(w0); }
    __device__ __forceinline__ void finish()
    {
        rotate(w0);
        for (int b = w0 + ROT_BATCH; b < w1; b += ROT_BATCH) {
            load(b);
            rotate(b);
        }
        wave_lds_fence();
    }
};

// The same rotations shared by the four waves of a workgroup, which then stream four column
// groups of the same (unit, projection, k-split): wave w rotates chunks w, w + 4, ... of the
// window into the workgroup's LDS rows and stores each chunk's sum; after a barrier every wave
// adds the sums in chunk order (the order of the per-wave stage, so the results are the same).
constexpr int ROT_WAVES = 4;

template <int TM, int NW = ROT_WAVES>
struct RotStageGroup {
    static constexpr bool kWork = true;
    static constexpr int NJ = ROT_CW / NW;            // chunks per wave and window
    const MoeParams& p;
    const int (&so)[TM];
    int tm, w0, w1, row_words, lane, wave;
    __amdgpu_buffer_rsrc_t suh_rsrc, x_rsrc[TM];
    uint32_t* dst;                                      // LDS rows
    float* sums;                                        // LDS [TM][ROT_CW] chunk sums
    float (&xs)[TM];
    uint32_t xv[TM][NJ], sv[NJ];

    __device__ __forceinline__ int chunk(int i) const { return min(w0 + wave + NW * i, w1 - 1); }
    __device__ __forceinline__ void issue()
    {
#pragma unroll
        for (int i = 0; i < NJ; ++i) sv[i] = __builtin_amdgcn_raw_buffer_load_b32(suh_rsrc, 4 * lane, 256 * chunk(i), 0);
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int i = 0; i < NJ; ++i) xv[m][i] = __builtin_amdgcn_raw_buffer_load_b32(x_rsrc[m], 4 * lane, 256 * chunk(i), 0);
    }
    __device__ __forceinline__ void finish()
    {
        const int slots = p.T * p.topk;
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m >= tm) continue;
            const bool shared = so[m] >= slots;
#pragma unroll
            for (int i = 0; i < NJ; ++i) {
                const int c = w0 + wave + NW * i;
                if (c < w1) {
                    const half2_t su = __builtin_bit_cast(half2_t, sv[i]);
                    float v0 = x_elem(xv[m][i], 0, p.x_dtype) * h2f(su.x);
                    float v1 = x_elem(xv[m][i], 1, p.x_dtype) * h2f(su.y);
                    if (shared) {
                        v0 = h2f(f2h(v0));
                        v1 = h2f(f2h(v1));
                    }
                    had128_pair(v0, v1, lane);
                    const half2_t r = {f2h(v0), f2h(v1)};
                    dst[m * row_words + (c - w0) * 64 + lane] = __builtin_bit_cast(uint32_t, r);
                    const float sm = wave_sum(h2f(r.x) + h2f(r.y));
                    if (lane == 0) sums[m * ROT_CW + (c - w0)] = sm;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < TM; ++m)
            if (m < tm)
                for (int c = 0; c < w1 - w0; ++c) xs[m] += sums[m * ROT_CW + c];
    }
};

// Gate/up GEMV of tm rows (slots slot[0..tm)) over the 128-chunks [c0, c1): each window of at
// most ROT_CW chunks is rotated into LDS (GROUP: by the workgroup's four waves together), then
// streamed; writes the fp32 partials of the rows.
template <int K2, int TM, bool GROUP, int NW = ROT_WAVES>
__device__ __forceinline__ void gate_up_rot_rows(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                 const int (&so)[TM], int tm, int cg, int c0, int c1, float* part,
                                                 uint32_t* lds, float* lsums)
{
    const int lane = threadIdx.x & 63;
    float acc[TM][2], xs[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) acc[m][0] = acc[m][1] = xs[m] = 0.0f;
    constexpr int RW = ROT_CW * 64;
    const int slots = p.T * p.topk;
    __amdgpu_buffer_rsrc_t xrs[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        const int row = so[m] >= slots ? so[m] - slots : so[m] / p.topk;
        xrs[m] = weight_rsrc((const uint32_t*)((const uint16_t*)p.x + (size_t)row * p.x_stride));
    }
    const __amdgpu_buffer_rsrc_t srs = weight_rsrc((const uint32_t*)suh);
    auto window = [&](int w0, int w1) {
        const XLds src{lds, RW, 8 * w0};
        if constexpr (GROUP) {
            RotStageGroup<TM, NW> stage{p, so, tm, w0, w1, RW, lane, (int)(threadIdx.x >> 6), srs, {}, lds, lsums, xs};
#pragma unroll
            for (int m = 0; m < TM; ++m) stage.x_rsrc[m] = xrs[m];
            gemv_wave<K2, TM>(trellis, p.I / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
        } else {
            RotStage<TM> stage{p, so, tm, w0, w1, RW, lane, srs, {}, lds, xs};
#pragma unroll
            for (int m = 0; m < TM; ++m) stage.x_rsrc[m] = xrs[m];
            gemv_wave<K2, TM>(trellis, p.I / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
        }
    };
    if (c1 - c0 <= ROT_CW) {
        window(c0, c1);                 // the common case, straight-line
    } else {
        for (int w0 = c0; w0 < c1; w0 += ROT_CW) {
            window(w0, min(c1, w0 + ROT_CW));
            // this window's reads before the next window's writes
            if constexpr (GROUP) __syncthreads();
            else wave_lds_fence();
        }
    }
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        if (m < tm) {
            float* dst = part + (size_t)so[m] * p.I;
            dst[col0] = MUL1_K_INV * acc[m][0] + MUL1_K_BIAS * xs[m];
            dst[col1] = MUL1_K_INV * acc[m][1] + MUL1_K_BIAS * xs[m];
        }
    }
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

template <int K2, int TM, bool GROUP>
__device__ __forceinline__ void gate_up_rot_rec(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                const int* slot, int tm, int cg, int c0, int c1, float* part,
                                                uint32_t* lds, float* lsums)
{
    int so[TM];
    record_slots<TM>(slot, tm, so);
    gate_up_rot_rows<K2, TM, GROUP>(p, trellis, suh, so, tm, cg, c0, c1, part, lds, lsums);
}

template <int K2, int TMAX, bool GROUP>
__device__ __forceinline__ void gate_up_rot_item(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                 const int* slot, int rows, int cg, int c0, int c1, float* part,
                                                 uint32_t* lds, float* lsums)
{
    if (rows <= TMAX) {                 // the common case, straight-line
        if constexpr (TMAX == 1) gate_up_rot_rec<K2, 1, GROUP>(p, trellis, suh, slot, rows, cg, c0, c1, part, lds, lsums);
        else if (rows <= 1) gate_up_rot_rec<K2, 1, GROUP>(p, trellis, suh, slot, rows, cg, c0, c1, part, lds, lsums);
        else gate_up_rot_rec<K2, 2, GROUP>(p, trellis, suh, slot, rows, cg, c0, c1, part, lds, lsums);
        return;
    }
    // a chunk of more than TMAX rows (given routes that repeat an expert) runs TMAX rows at a time
    for (int r0 = 0; r0 < rows; r0 += TMAX) {
        const int tr = rows - r0 < TMAX ? rows - r0 : TMAX;
        if constexpr (TMAX == 1) gate_up_rot_rec<K2, 1, GROUP>(p, trellis, suh, slot + r0, tr, cg, c0, c1, part, lds, lsums);
        else {
            static_assert(TMAX == 2, "decode path rows: 1 or 2");
            if (tr <= 1) gate_up_rot_rec<K2, 1, GROUP>(p, trellis, suh, slot + r0, tr, cg, c0, c1, part, lds, lsums);
            else gate_up_rot_rec<K2, 2, GROUP>(p, trellis, suh, slot + r0, tr, cg, c0, c1, part, lds, lsums);
        }
        if constexpr (GROUP) __syncthreads();      // this pass's LDS reads before the next pass's writes
        else wave_lds_fence();
    }
}

// One wave per (unit, gate|up, k-split, 128 columns). GROUP (the column-group count a multiple
// of 4): the items run column group fastest, so the four waves of a workgroup share unit,
// projection and k-split (and exit together) and rotate their inputs together; otherwise every
// wave rotates its own.
template <int TMAX, bool GROUP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void moe_gate_up_rot_kernel(MoeParams p)
{
    __shared__ uint32_t xl[GROUP ? 1 : 4][TMAX * ROT_CW * 64];
    __shared__ float xsums[TMAX * ROT_CW];
    const int wave = threadIdx.x >> 6;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.I / 128;
    const KSplit k = ks_gate_up(p, p.units_max);
    const int per_unit = 2 * ncg * k.base;
    const int u = __builtin_amdgcn_readfirstlane(wid / per_unit);
    if (u >= p.units_max) return;
    const UnitRec* rp = p.urec + u;
    const int e = __builtin_amdgcn_readfirstlane(rp->e);
    if (e == EVAMX_NO_UNIT) return;
    const int ubase = __builtin_amdgcn_readfirstlane(rp->ubase);
    const int S = __builtin_amdgcn_readfirstlane(rp->s_gu);
    const int r = wid - ubase * per_unit;
    if (r >= 2 * ncg * S) return;
    int cg, proj, ks;
    if constexpr (GROUP) {
        cg = __builtin_amdgcn_readfirstlane(r % ncg);
        const int pk = r / ncg;
        proj = __builtin_amdgcn_readfirstlane(pk / S);
        ks = __builtin_amdgcn_readfirstlane(pk % S);
    } else {
        cg = __builtin_amdgcn_readfirstlane(r / (2 * S));
        const int rem = r % (2 * S);
        proj = __builtin_amdgcn_readfirstlane(rem / S);
        ks = __builtin_amdgcn_readfirstlane(rem % S);
    }
    const int rows = __builtin_amdgcn_readfirstlane(rp->rows);
    const int k2 = __builtin_amdgcn_readfirstlane(rp->k2);
    const int nch = p.H / 128;
    const int c0 = nch * ks / S, c1 = nch * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)rp->tr[proj];
    const half_t* suh = (const half_t*)rp->suh[proj];
    float* part = p.part_gu + ((size_t)ks * 2 + proj) * moe_nslot(p) * p.I;
    uint32_t* lds = xl[GROUP ? 0 : wave];
    switch (k2) {
        case 3: gate_up_rot_item<3, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 4: gate_up_rot_item<4, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 5: gate_up_rot_item<5, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 6: gate_up_rot_item<6, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 7: gate_up_rot_item<7, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 8: gate_up_rot_item<8, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        case 10: gate_up_rot_item<10, TMAX, GROUP>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); break;
        default: {
            // unsupported rate (flagged by the prepare): zero partials, so no output reads stale data
            const int lane = threadIdx.x & 63;
            for (int m = 0; m < rows; ++m) {
                float* dst = part + (size_t)rp->slot[m] * p.I + cg * 128;
                dst[lane_col(lane, 0)] = 0.0f;
                dst[lane_col(lane, 1)] = 0.0f;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// One-row calls route inside the gate/up launch (no prepare launch). Units are the routed slots
// in slot order, then the shared expert: unit j is slot j, so a gate/up wave knows its slot from
// its unit alone. Each routed wave routes the token itself (every wave computes the same routes)
// and reads its expert's pointers; the shared expert's waves start streaming at once. The grid's
// extra last workgroup publishes what moe_prepare_gemv_kernel publishes for the later stages and
// the caller: routes, local experts, the run table and order, the unit and slot records, meta.

// The expert and fp16 routing weight of slot j of the one-row call, in lane j < topk.
__device__ __forceinline__ void slot_routes1(const MoeParams& p, int lane, int& id, half_t& rw, float& w32)
{
    id = -1;
    rw = f2h(0.0f);
    w32 = 0.0f;
    if (p.logits) {
        route_lanes(p, 0, lane, id, w32);
        rw = f2h(w32);
    } else if (lane < p.topk) {
        const int64_t e = p.sel[lane];
        // indices outside the int range are outside any table: keep them out of range
        id = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
        rw = p.weights ? f2h(p.weights[lane]) : p.rw16[lane];
    }
}

__device__ __forceinline__ void publish_routes1(const MoeParams& p, int lane)
{
    const int topk = p.topk;                       // slots 0..topk-1; the shared row is slot topk
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = lane; i < table_len; i += 64) p.runs[i] = 0;
    }
    int id;
    half_t rw;
    float w32;
    slot_routes1(p, lane, id, rw, w32);
    int e = -1;
    if (lane < topk) {
        if (p.logits) {
            p.sel[lane] = id;
            p.weights[lane] = w32;
            p.rw16[lane] = rw;
        } else if (p.weights) {
            p.rw16[lane] = rw;
        }
        e = slot_local(p, id, rw, true);
        p.local[lane] = e;
    }
    // unit and slot records: lane j < topk for slot j, lane topk for the shared expert
    const int sgu = ks_of_chunk(ks_gate_up(p, p.units_max), 1), sd = ks_of_chunk(ks_down(p, p.units_max), 1);
    const bool sh_lane = p.has_shared && lane == topk;
    if (lane < topk || sh_lane) {
        SlotRec q = {};
        UnitRec r = {};
        r.e = EVAMX_NO_UNIT;
        if (sh_lane || e >= 0) {
            const int ex = sh_lane ? -1 : e;
            auto ptr = [&](int row) -> uint64_t {
                return sh_lane ? (uint64_t)p.sh_ptr[row] : (uint64_t)p.tables[(size_t)row * p.tbl_stride + e];
            };
            const int k2 = k2_gu_of(p, ex), k2d = k2_d_of(p, ex);
            if (!gemv_k2_supported(k2) || !gemv_k2_supported(k2d)) atomicOr(p.err, EVAMX_ERR_RATE);
            q.active = 1;
            q.shared = sh_lane ? 1 : 0;
            q.s_gu = sgu;
            q.s_d = sd;
            q.w = sh_lane ? 1.0f : h2f(rw);
            q.g_svh = ptr(EVAMX_TBL_G_SVH);
            q.u_svh = ptr(EVAMX_TBL_U_SVH);
            q.d_suh = ptr(EVAMX_TBL_D_SUH);
            q.d_svh = ptr(EVAMX_TBL_D_SVH);
            r.e = ex;
            r.rows = 1;
            r.k2 = k2;
            r.ubase = lane;
            r.s_gu = sgu;
            r.s_d = sd;
            r.k2_d = k2d;
#pragma unroll
            for (int j = 0; j < EVAMX_CHUNK; ++j) r.slot[j] = lane;
            r.tr[0] = ptr(EVAMX_TBL_G_TRELLIS);
            r.tr[1] = ptr(EVAMX_TBL_U_TRELLIS);
            r.tr[2] = ptr(EVAMX_TBL_D_TRELLIS);
            r.suh[0] = ptr(EVAMX_TBL_G_SUH);
            r.suh[1] = ptr(EVAMX_TBL_U_SUH);
        }
        p.srec[lane] = q;
        p.urec[lane] = r;
    }
    // the run table's zeros (other lanes) complete before its entries are written
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // stable grouping by (expert, slot), as moe_prepare_gemv_kernel
    const uint32_t key = wave_sort_asc(e >= 0 ? ((uint32_t)e << 6) | (uint32_t)lane : 0xffffffffu, lane);
    const bool act = key != 0xffffffffu;
    const int ge = (int)(key >> 6), gs = (int)(key & 63);
    const int n_active = __popcll(__ballot(act));
    const int prev_e = __shfl_up(ge, 1, WAVE);
    const uint64_t heads = __ballot(act && (lane == 0 || prev_e != ge));
    const uint64_t le_mask = lane == 63 ? ~0ull : ((2ull << lane) - 1);
    const int first = 63 - __clzll(heads & le_mask);
    const bool rs = act && ((lane - first) % EVAMX_CHUNK) == 0;
    const uint64_t rmask = __ballot(rs);
    const int n_runs = __popcll(rmask);
    if (act) {
        if (p.runs) {
            p.runs[2 + p.slots_max + 1 + lane] = gs;
            if (rs) p.runs[2 + __popcll(rmask & (le_mask >> 1))] = lane;
        }
        p.order[lane] = gs;
    }
    if (lane == 0) {
        if (p.has_shared) p.order[n_active] = topk;
        if (p.runs) {
            p.runs[0] = n_runs;
            p.runs[1] = 0;
            p.runs[2 + n_runs] = n_active;
        }
        p.meta[0] = n_runs + (p.has_shared ? 1 : 0);
        p.meta[1] = n_active;
        p.meta[2] = topk + (p.has_shared ? 1 : 0);
        p.meta[3] = 0;
    }
}

template <bool GROUP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void moe_gate_up_route1_kernel(MoeParams p)
{
    __shared__ uint32_t xl[GROUP ? 1 : 4][ROT_CW * 64];
    __shared__ float xsums[ROT_CW];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (blockIdx.x == gridDim.x - 1) {
        if (wave == 0) publish_routes1(p, lane);
        return;
    }
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.I / 128;
    const int S = ks_of_chunk(ks_gate_up(p, p.units_max), 1);
    const int per_unit = 2 * ncg * S;
    const int u = __builtin_amdgcn_readfirstlane(wid / per_unit);
    if (u >= p.units_max) return;
    const int r = wid - u * per_unit;
    int cg, proj, ks;
    if constexpr (GROUP) {
        cg = __builtin_amdgcn_readfirstlane(r % ncg);
        const int pk = r / ncg;
        proj = __builtin_amdgcn_readfirstlane(pk / S);
        ks = __builtin_amdgcn_readfirstlane(pk % S);
    } else {
        cg = __builtin_amdgcn_readfirstlane(r / (2 * S));
        const int rem = r % (2 * S);
        proj = __builtin_amdgcn_readfirstlane(rem / S);
        ks = __builtin_amdgcn_readfirstlane(rem % S);
    }
    int e = -1;                                   // the shared expert's unit (u == topk)
    if (u < p.topk) {
        int id;
        half_t rw;
        float w32;
        slot_routes1(p, lane, id, rw, w32);
        id = __builtin_amdgcn_readlane(id, u);
        const half_t rwu = __builtin_bit_cast(half_t, (uint16_t)__builtin_amdgcn_readlane((int)__builtin_bit_cast(uint16_t, rw), u));
        e = __builtin_amdgcn_readfirstlane(slot_local(p, id, rwu, false));
        if (e < 0) return;                        // inactive slot: no partials are read
    }
    const int k2 = __builtin_amdgcn_readfirstlane(k2_gu_of(p, e));
    // constant table rows (a row index that depends on proj would put the kernel argument's
    // shared-pointer array in scratch memory to index it)
    const uint32_t* trellis = (const uint32_t*)(proj == 0 ? expert_ptr(p, e, EVAMX_TBL_G_TRELLIS)
                                                          : expert_ptr(p, e, EVAMX_TBL_U_TRELLIS));
    const half_t* suh = (const half_t*)(proj == 0 ? expert_ptr(p, e, EVAMX_TBL_G_SUH) : expert_ptr(p, e, EVAMX_TBL_U_SUH));
    const int nch = p.H / 128;
    const int c0 = nch * ks / S, c1 = nch * (ks + 1) / S;
    float* part = p.part_gu + ((size_t)ks * 2 + proj) * moe_nslot(p) * p.I;
    uint32_t* lds = xl[GROUP ? 0 : wave];
    const int so[1] = {u};                        // unit u is slot u (the shared row: slot topk)
    switch (k2) {
        case 3: gate_up_rot_rows<3, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 4: gate_up_rot_rows<4, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 5: gate_up_rot_rows<5, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 6: gate_up_rot_rows<6, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 7: gate_up_rot_rows<7, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 8: gate_up_rot_rows<8, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        case 10: gate_up_rot_rows<10, 1, GROUP>(p, trellis, suh, so, 1, cg, c0, c1, part, lds, xsums); break;
        default: {
            // unsupported rate (flagged by the publishing wave): zero partials
            float* dst = part + (size_t)u * p.I + cg * 128;
            dst[lane_col(lane, 0)] = 0.0f;
            dst[lane_col(lane, 1)] = 0.0f;
        }
    }
}

// Down GEMV of the decode path: one wave per (unit, 128 columns, k-split), from the unit's record.
template <int TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void moe_down_rec_kernel(MoeParams p)
{
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.H / 128;
    const KSplit k = ks_down(p, p.units_max);
    const int per_unit = ncg * k.base;
    const int u = __builtin_amdgcn_readfirstlane(wid / per_unit);
    if (u >= p.units_max) return;
    const UnitRec* rp = p.urec + u;
    const int e = __builtin_amdgcn_readfirstlane(rp->e);
    if (e == EVAMX_NO_UNIT) return;
    const int ubase = __builtin_amdgcn_readfirstlane(rp->ubase);
    const int S = __builtin_amdgcn_readfirstlane(rp->s_d);
    const int r = wid - ubase * per_unit;
    if (r >= ncg * S) return;
    const int cg = __builtin_amdgcn_readfirstlane(r / S), ks = __builtin_amdgcn_readfirstlane(r % S);
    const int rows = __builtin_amdgcn_readfirstlane(rp->rows);
    const int k2 = __builtin_amdgcn_readfirstlane(rp->k2_d);
    const int na = p.I / 128;
    const int c0 = na * ks / S, c1 = na * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)rp->tr[2];
    float* part = p.part_d + (size_t)ks * moe_nslot(p) * p.H;
    gemv_dispatch_k<TMAX>(k2, trellis, p.H / 16, cg, c0, c1, GlobalRows{p.act, (size_t)p.I, p.actsum, na}, rp->slot,
                          rows, part, (size_t)p.H);
}

// Fixed-order sums over the k-splits q = 0..S-1 of N values per lane, value n at
// base[n] + q * stride: each sum adds its splits in q order starting from 0, as a sequential
// loop does, but the loads of up to QB splits of all N values are issued before any of their
// adds (one memory round trip per QB splits instead of one per split and value). S is
// wave-uniform; splits past S are neither loaded nor added.
template <int N, int QB>
__device__ __forceinline__ void sum_splits(const float* const (&base)[N], size_t stride, int S, float (&acc)[N])
{
#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = 0.0f;
    for (int q0 = 0; q0 < S; q0 += QB) {
        float t[N][QB];
#pragma unroll
        for (int i = 0; i < QB; ++i)
            if (q0 + i < S)
#pragma unroll
                for (int n = 0; n < N; ++n) t[n][i] = gptr<float>(base[n])[(size_t)(q0 + i) * stride];
#pragma unroll
        for (int i = 0; i < QB; ++i)
            if (q0 + i < S)
#pragma unroll
                for (int n = 0; n < N; ++n) acc[n] += t[n][i];
    }
}

// Activation epilogue: one wave per (grouped row o, 128-chunk a of I). Sums the gate/up
// partials in fixed order, rounds to fp16 (gu_f32 = false), then exl3_moe_coop_kernel.cuh:
// 784-805 for routed slots (act_gate with the clamp after SiLU) or the shared expert's EXL3
// linear outputs + swiglu (model.py:450-452, kernels.py:213-217), and the down projection's
// input rotation; writes act (fp16) and the chunk's sum.
// REC (decode path): waves are (slot, chunk group), every slot's work resolved from its record
// (inactive slots exit); otherwise (grouped row, chunk group) over the call's active rows.
template <int CPW, bool REC>
__global__ __launch_bounds__(256) void moe_act_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int na = p.I / 128;
    const int ng = na / CPW;                 // chunk groups per row (CPW divides na)
    int o, a0;
    if (!REC && p.act_class) {
        // one size class of the MFMA tiles: wave -> (tile of the class, row of the tile up to the
        // class's row bound, chunk group); rows past the tile's exit at once
        const int cap = p.act_class == 1 ? EVAMX_SMALL_TILE_ROWS : EVAMX_TILE_ROWS;
        const int n_small = __builtin_amdgcn_readfirstlane(p.meta[3]);
        const int n_cls = p.act_class == 1 ? n_small : __builtin_amdgcn_readfirstlane(p.meta[0]) - n_small;
        const int ti = wid / (cap * ng);
        if (ti >= n_cls) return;
        const int rem = wid - ti * cap * ng;
        const int r = rem / ng;
        a0 = (rem % ng) * CPW;
        const int tile = __builtin_amdgcn_readfirstlane(p.act_class == 1 ? p.tiles[ti] : p.tiles[p.max_chunks - 1 - ti]);
        const int* ch = p.chunks + 8 * tile;
        if (r >= __builtin_amdgcn_readfirstlane(ch[2])) return;
        o = __builtin_amdgcn_readfirstlane(ch[1]) + r;
    } else {
        const int n_rows = REC ? moe_nslot(p) : p.meta[1] + (p.has_shared ? p.T : 0);
        if (wid >= n_rows * ng) return;
        o = wid / ng;
        a0 = (wid % ng) * CPW;
    }
    int s, Sg;
    bool shared;
    const half_t *g_svh, *u_svh, *d_suh;
    if constexpr (REC) {
        s = o;
        const SlotRec* rp = p.srec + s;
        if (!__builtin_amdgcn_readfirstlane(rp->active)) return;
        shared = __builtin_amdgcn_readfirstlane(rp->shared) != 0;
        Sg = __builtin_amdgcn_readfirstlane(rp->s_gu);
        g_svh = (const half_t*)rp->g_svh;
        u_svh = (const half_t*)rp->u_svh;
        d_suh = (const half_t*)rp->d_suh;
    } else {
        const int slots = p.T * p.topk;
        s = __builtin_amdgcn_readfirstlane(p.order[o]);
        const int e = s < slots ? __builtin_amdgcn_readfirstlane(p.local[s]) : -1;
        shared = e < 0;
        g_svh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_G_SVH);
        u_svh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_U_SVH);
        d_suh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_D_SUH);
        Sg = ks_of_chunk(ks_gate_up(p, __builtin_amdgcn_readfirstlane(p.meta[2])),
                         __builtin_amdgcn_readfirstlane(p.slot_mult[s]));
    }
    const float L = p.limit;
    const int nslot = moe_nslot(p);
    if (shared && a0 == 0 && p.sh_gate_w) {
        // gated shared expert: the row's scale sigmoid(x . w), fp32 dot of the fp16 row
        // (exl3_moe_coop_kernel.cuh:881-903), for the combine stage
        const int row = s - p.T * p.topk;
        const uint32_t* xw = (const uint32_t*)((const uint16_t*)p.x + (size_t)row * p.x_stride);
        const uint32_t* ww = (const uint32_t*)p.sh_gate_w;
        float d = 0.0f;
        for (int i = lane; i < p.H / 2; i += 64) {
            const uint32_t xv = xw[i];
            const half2_t wv = __builtin_bit_cast(half2_t, ww[i]);
            d = fmaf(x_elem(xv, 0, p.x_dtype), h2f(wv.x), d);
            d = fmaf(x_elem(xv, 1, p.x_dtype), h2f(wv.y), d);
        }
        d = wave_sum(d);
        if (lane == 0) p.gate_val[row] = 1.0f / (1.0f + __expf(-d));
    }
    // all chunks' scales and partial sums first, so their loads are in flight together
    float g[CPW][2], u[CPW][2], gs[CPW][2], us[CPW][2], ds[CPW][2];
    const float* base[4 * CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = (a0 + c) * 128 + lane_col(lane, h);
            gs[c][h] = h2f(g_svh[col]);
            us[c][h] = h2f(u_svh[col]);
            ds[c][h] = h2f(d_suh[col]);
            base[4 * c + h] = p.part_gu + (size_t)s * p.I + col;                          // gate
            base[4 * c + 2 + h] = p.part_gu + (size_t)(nslot + s) * p.I + col;            // up
        }
    }
    float sums[4 * CPW];
    sum_splits<4 * CPW, CPW == 1 ? 8 : 2>(base, (size_t)2 * nslot * p.I, Sg, sums);
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            g[c][h] = sums[4 * c + h];
            u[c][h] = sums[4 * c + 2 + h];
        }
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        float gg[2], uu[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            gg[h] = h2f(f2h(g[c][h]));     // GEMV output stored as fp16 (gu_f32 = false)
            uu[h] = h2f(f2h(u[c][h]));
        }
        had128_lane(gg[0], gg[1], lane);
        had128_lane(uu[0], uu[1], lane);
        float av[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (shared) {
                // EXL3 linear outputs: fp16 after the rotation, fp16 product with svh; swiglu
                // clamps the gate BEFORE SiLU; mid to fp16; fp16 product with the down suh
                float gv = h2f(f2h(h2f(f2h(gg[h])) * gs[c][h]));
                float uv = h2f(f2h(h2f(f2h(uu[h])) * us[c][h]));
                if (L > 0.0f) {
                    // torch.clamp: a NaN stays NaN (fminf/fmaxf would return the limit)
                    uv = uv < -L ? -L : (uv > L ? L : uv);
                    gv = gv > L ? L : gv;
                }
                const float mid = h2f(f2h(silu_f(gv) * uv));
                av[h] = h2f(f2h(mid * ds[c][h]));
            } else {
                const float gv = gg[h] * gs[c][h];
                float uv = uu[h] * us[c][h];
                float x = silu_f(gv);
                if (L != 0.0f) {
                    // fminf/fmaxf as the reference kernel: a NaN operand yields the limit
                    uv = fminf(fmaxf(uv, -L), L);
                    x = fminf(x, L);
                }
                av[h] = x * uv * ds[c][h];
            }
        }
        had128_lane(av[0], av[1], lane);
        half_t* dst = p.act + (size_t)s * p.I + (a0 + c) * 128;
        const half_t r0 = f2h(av[0]), r1 = f2h(av[1]);
        dst[lane_col(lane, 0)] = r0;
        dst[lane_col(lane, 1)] = r1;
        const float sum = wave_sum(h2f(r0) + h2f(r1));
        if (lane == 0) p.actsum[(size_t)s * na + a0 + c] = sum;
    }
}

// The activation stage for the rows of one size class of MFMA tiles (cls 1: tiles of at most 16
// rows, cls 2: larger), calls of more than 16 tokens.
static void launch_act_class(const MoeParams& p, int cls, hipStream_t stream)
{
    const int na = p.I / 128;
    MoeParams q = p;
    q.act_class = cls;
    const long cap = cls == 1 ? EVAMX_SMALL_TILE_ROWS : EVAMX_TILE_ROWS;
    if (p.T > EVAMX_SMALL_ROWS && na % 4 == 0) {
        const long waves = (long)p.max_chunks * cap * (na / 4);
        launch_timed(moe_act_kernel<4, false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), stream, nullptr, nullptr, q);
    } else {
        const long waves = (long)p.max_chunks * cap * na;
        launch_timed(moe_act_kernel<1, false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), stream, nullptr, nullptr, q);
    }
}

// Activation launch: one wave per (row, chunk) for small batches (latency), per (row, 4 chunks)
// for large ones (the row's slot, expert and pointers resolved once).
static void launch_act(const MoeParams& p, int nslot, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const int na = p.I / 128;
    if (p.T <= EVAMX_GEMV_MAX_ROWS) {
        const int waves = nslot * na;
        launch_timed(moe_act_kernel<1, true>, dim3((waves + 3) / 4), dim3(256), stream, start, stop, p);
    } else if (p.T > EVAMX_SMALL_ROWS && na % 4 == 0) {
        const int waves = nslot * (na / 4);
        launch_timed(moe_act_kernel<4, false>, dim3((waves + 3) / 4), dim3(256), stream, start, stop, p);
    } else {
        const int waves = nslot * na;
        launch_timed(moe_act_kernel<1, false>, dim3((waves + 3) / 4), dim3(256), stream, start, stop, p);
    }
}

// Sum of the down k-split partials of slot s on this lane's two columns, fixed order; loads of
// four splits are issued before their adds. (sum_splits here was slower in the combine
// kernels: 9.2 -> 9.9 us at 16 tokens, 85 -> 110 us at 512.)
__device__ __forceinline__ void sum_partials(const MoeParams& p, int s, int cg, int lane, int S, float (&v)[2])
{
    const size_t stride = (size_t)moe_nslot(p) * p.H;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float* pp = p.part_d + (size_t)s * p.H + cg * 128 + lane_col(lane, h);
        float acc = 0.0f;
        int q = 0;
        for (; q + 4 <= S; q += 4) {
            float t[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) t[i] = pp[(q + i) * stride];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc += t[i];
        }
        for (; q < S; ++q) acc += pp[q * stride];
        v[h] = acc;
    }
}

// Output rotation * svh * weight of one item's summed down partials: routed slots in fp32;
// the shared expert with the EXL3 linear's fp16 rounding points (C in fp16, fp16 svh product).
__device__ __forceinline__ void combine_item(bool shared, float w, float s0, float s1, float (&v)[2], int lane)
{
    if (shared) {
        v[0] = h2f(f2h(v[0]));
        v[1] = h2f(f2h(v[1]));
    }
    had128_lane(v[0], v[1], lane);
    if (shared) {
        v[0] = h2f(f2h(h2f(f2h(v[0])) * s0));
        v[1] = h2f(f2h(h2f(f2h(v[1])) * s1));
    } else {
        v[0] = w * (v[0] * s0);
        v[1] = w * (v[1] * s1);
    }
}

__device__ __forceinline__ void combine_store(const MoeParams& p, int row, int col0, int col1, float o0, float o1)
{
    if (p.out) {
        float* dst = p.out + (size_t)row * p.out_stride;
        dst[col0] = o0;
        dst[col1] = o1;
    }
    if (p.residual) {
        // h = bf16(h + bf16(y)): y cast to the activation dtype, then the bf16 add
        uint16_t* h = p.residual + (size_t)row * p.residual_stride;
        h[col0] = bf16_bits(bf16_value(h[col0]) + bf16_value(bf16_bits(o0)));
        h[col1] = bf16_bits(bf16_value(h[col1]) + bf16_value(bf16_bits(o1)));
    }
}

// Per-token reduction over slots in slot order (+ shared expert), for small batches: one
// workgroup per (token, 128 columns) with one wave per item (slot or shared expert;
// grid-stride when there are more items than waves) into LDS, then wave 0 sums them in slot
// order, as the reference sums one warp per slot (exl3_moe_coop_kernel.cuh:906-940), and adds
// the shared expert. A wave issues its item's independent loads (expert, weight, split count)
// together, then the svh pointer and the partials, so an item costs two memory round trips.
constexpr int EVAMX_COMBINE_WAVES = 16;

// REC (decode path): an item's activity, weight, split count and svh come from its slot record.
template <bool REC>
__global__ __launch_bounds__(64 * EVAMX_COMBINE_WAVES) void moe_combine_kernel(MoeParams p)
{
    __shared__ float part[EVAMX_MAX_TOPK + 1][128];
    __shared__ int active[EVAMX_MAX_TOPK + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int ncg = p.H / 128;
    const int row = blockIdx.x / ncg, cg = blockIdx.x % ncg;
    const int slots = p.T * p.topk;
    const int c0 = lane_col(lane, 0), c1 = lane_col(lane, 1);
    const int col0 = cg * 128 + c0, col1 = cg * 128 + c1;
    const int nitems = p.topk + (p.has_shared ? 1 : 0);
    for (int k = wave; k < nitems; k += nw) {
        const bool shared = k == p.topk;
        const int sk = shared ? slots + row : row * p.topk + k;
        float w;
        int S;
        const half_t* svh;
        if constexpr (REC) {
            const SlotRec* rp = p.srec + sk;
            if (!__builtin_amdgcn_readfirstlane(rp->active)) {
                if (lane == 0) active[k] = 0;
                continue;
            }
            w = rp->w;
            S = __builtin_amdgcn_readfirstlane(rp->s_d);
            svh = (const half_t*)rp->d_svh;
        } else {
            const int le = shared ? -1 : __builtin_amdgcn_readfirstlane(p.local[sk]);
            const int mult = __builtin_amdgcn_readfirstlane(p.slot_mult[sk]);
            const int units = __builtin_amdgcn_readfirstlane(p.meta[2]);
            w = shared ? 1.0f : h2f(p.rw16[sk]);
            if (!shared && le < 0) {
                if (lane == 0) active[k] = 0;
                continue;
            }
            svh = shared ? (const half_t*)p.sh_ptr[EVAMX_TBL_D_SVH]
                         : (const half_t*)p.tables[(size_t)EVAMX_TBL_D_SVH * p.tbl_stride + le];
            S = ks_of_chunk(ks_down(p, units), mult);
        }
        float v[2];
        sum_partials(p, sk, cg, lane, S, v);
        combine_item(shared, w, h2f(svh[col0]), h2f(svh[col1]), v, lane);
        if (shared && p.sh_gate_w) {
            // gated shared expert: gv * shared (exl3_moe_coop_kernel.cuh:942-948)
            const float gv = p.gate_val[row];
            v[0] = gv * v[0];
            v[1] = gv * v[1];
        }
        part[k][c0] = v[0];
        part[k][c1] = v[1];
        if (lane == 0) active[k] = 1;
    }
    __syncthreads();
    if (wave == 0) {
        float o0 = 0.0f, o1 = 0.0f;
        for (int k = 0; k < p.topk; ++k) {
            if (!active[k]) continue;
            o0 = o0 + part[k][c0];
            o1 = o1 + part[k][c1];
        }
        if (p.has_shared) {
            o0 = o0 + part[p.topk][c0];
            o1 = o1 + part[p.topk][c1];
        }
        combine_store(p, row, col0, col1, o0, o1);
    }
}

// The same reduction for large batches, where throughput matters more than the latency of one
// token: one wave per (token, CGW groups of 128 columns) walks the token's items in slot order
// (shared expert last), COMBINE_BATCH items at a time: it reads their metadata (local expert,
// split count, weight, svh pointer) once for its CGW column groups, then for each column group
// issues the items' loads together and adds them in slot order. Same operations in the same order
// per column as moe_combine_kernel, so the two give identical results.
constexpr int COMBINE_BATCH = 4;

template <int CGW>
__global__ __launch_bounds__(256) void moe_combine_rows_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    const int ngw = p.H / 128 / CGW;                 // column-group blocks per token (CGW divides H/128)
    if (wid >= p.T * ngw) return;
    const int row = wid / ngw, cg0 = (wid - row * ngw) * CGW;
    const int slots = p.T * p.topk;
    const KSplit kd = ks_down(p, __builtin_amdgcn_readfirstlane(p.meta[2]));
    const int nitems = p.topk + (p.has_shared ? 1 : 0);
    float o[CGW][2];
#pragma unroll
    for (int c = 0; c < CGW; ++c) o[c][0] = o[c][1] = 0.0f;
    for (int b = 0; b < nitems; b += COMBINE_BATCH) {
        int sk[COMBINE_BATCH], le[COMBINE_BATCH], S[COMBINE_BATCH];
        float w[COMBINE_BATCH];
        const half_t* svh[COMBINE_BATCH];
#pragma unroll
        for (int j = 0; j < COMBINE_BATCH; ++j) {
            const int k = b + j;
            const bool shared = k == p.topk;
            sk[j] = shared ? slots + row : row * p.topk + k;
            le[j] = -2;                                   // -2: past the items
            svh[j] = nullptr;
            if (k < nitems) {
                le[j] = shared ? -1 : __builtin_amdgcn_readfirstlane(p.local[sk[j]]);
                S[j] = ks_of_chunk(kd, __builtin_amdgcn_readfirstlane(p.slot_mult[sk[j]]));
                w[j] = shared ? 1.0f : h2f(p.rw16[sk[j]]);
                if (le[j] >= 0 || (shared && le[j] == -1))
                    svh[j] = shared ? (const half_t*)p.sh_ptr[EVAMX_TBL_D_SVH]
                                    : (const half_t*)p.tables[(size_t)EVAMX_TBL_D_SVH * p.tbl_stride + le[j]];
            }
        }
#pragma unroll
        for (int c = 0; c < CGW; ++c) {
            const int cg = cg0 + c;
            const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
            float v[COMBINE_BATCH][2], sv[COMBINE_BATCH][2];
#pragma unroll
            for (int j = 0; j < COMBINE_BATCH; ++j) {
                if (svh[j]) {
                    sum_partials(p, sk[j], cg, lane, S[j], v[j]);
                    sv[j][0] = h2f(svh[j][col0]);
                    sv[j][1] = h2f(svh[j][col1]);
                }
            }
#pragma unroll
            for (int j = 0; j < COMBINE_BATCH; ++j) {
                if (svh[j]) {
                    const bool shared = b + j == p.topk;
                    combine_item(shared, w[j], sv[j][0], sv[j][1], v[j], lane);
                    if (shared && p.sh_gate_w) {
                        const float gv = p.gate_val[row];
                        v[j][0] = gv * v[j][0];
                        v[j][1] = gv * v[j][1];
                    }
                    o[c][0] = o[c][0] + v[j][0];
                    o[c][1] = o[c][1] + v[j][1];
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < CGW; ++c)
        combine_store(p, row, (cg0 + c) * 128 + lane_col(lane, 0), (cg0 + c) * 128 + lane_col(lane, 1), o[c][0], o[c][1]);
}

// ---------------------------------------------------------------------------------------------
// Host side.

int moe_prepare_only(MoeParams& p, hipStream_t stream)
{
    if (p.logits) hipLaunchKernelGGL(moe_route_kernel, dim3((p.T + 3) / 4), dim3(256), 0, stream, p);
    if (p.mode & PREP_GROUP) hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(64 * GROUP_WAVES), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_router_logits(const MoeParams& p, float* logits, hipStream_t stream)
{
    const int waves = p.n_logits * ((p.T + GATE_ROWS - 1) / GATE_ROWS);
    hipLaunchKernelGGL(moe_gate_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p, logits);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

bool moe_small_path(int T, int topk) { return T * topk <= EVAMX_SMALL_SLOTS && T <= EVAMX_SMALL_ROWS; }

int moe_launch(MoeParams& p, hipStream_t stream, void* const* events)
{
    // events[2k] / events[2k + 1]: start of the first and end of the last kernel of stage k
    auto ev = [&](int i) { return events ? (hipEvent_t)events[i] : (hipEvent_t) nullptr; };
    const int nch = p.H / 128;
    const int nslot = p.T * p.topk + (p.has_shared ? p.T : 0);
    const bool small = moe_small_path(p.T, p.topk);
    p.mfma = p.T >= EVAMX_MFMA_MIN_ROWS ? 1 : 0;
    // up to 16 tokens only the 16-row MFMA kernel runs, so the tiles are cut at 16 rows (more
    // than 16 slots of one expert occur only when given routes repeat an expert within a token)
    p.chunk_rows = !p.mfma ? EVAMX_CHUNK : p.T <= EVAMX_SMALL_TILE_ROWS ? EVAMX_SMALL_TILE_ROWS : EVAMX_TILE_ROWS;
    // decode path: chunks of at most 8 rows weigh at most their row count, so the call has at
    // most one unit per slot plus the shared expert's one (its rows fit one chunk)
    p.units_max = p.T * p.topk + (p.has_shared ? 1 : 0);
    hipEvent_t first = ev(0);
    // one-row calls route inside the gate/up launch: their prepare stage is the router front
    // alone (given gate_w), else it has no kernel and records no events
    const bool route1 = !p.mfma && p.T == 1;
    if (p.gate_w) {
        const int waves = p.n_logits * ((p.T + GATE_ROWS - 1) / GATE_ROWS);
        launch_timed(moe_gate_kernel, dim3((waves + 3) / 4), dim3(256), stream, first, route1 ? ev(1) : nullptr, p,
                     const_cast<float*>(p.logits));
        first = nullptr;
    }
    if (route1) {
        // one-row calls: the gate/up launch routes (no prepare launch, no prepare events)
    } else if (!p.mfma) {
        // decode path: one workgroup routes, groups and writes the records; the gate/up waves
        // rotate their own inputs
        launch_timed(moe_prepare_gemv_kernel, dim3(1), dim3(256), stream, first, ev(1), p);
    } else if (small) {
        // workgroup 0 groups, the others rotate; a wave per token routes in every workgroup
        // at most one workgroup per CU (gemv_waves = 16 per CU), so that none waits for a slot
        const int nwv = p.T > 4 ? p.T : 4;
        const int cus = p.gemv_waves / 16 > 2 ? p.gemv_waves / 16 : 2;
        int blocks = 1 + (nslot * nch * 2 + nwv - 1) / nwv;
        if (blocks > cus) blocks = cus;
        launch_timed(moe_prepare_small_kernel, dim3(blocks), dim3(64 * nwv), stream, first, ev(1), p);
    } else {
        if (p.logits) {
            launch_timed(moe_route_kernel, dim3((p.T + 3) / 4), dim3(256), stream, first, nullptr, p);
            first = nullptr;
        }
        launch_timed(moe_group_kernel, dim3(1), dim3(64 * GROUP_WAVES), stream, first, nullptr, p);
        launch_timed(moe_rotate_kernel, dim3(EVAMX_ROTATE_BLOCKS), dim3(256), stream, nullptr, ev(1), p);
    }
    const SideStream* side = p.mfma && p.T > EVAMX_SMALL_TILE_ROWS && p.side_ok && !events
                                 ? side_stream(stream) : nullptr;
    if (side) {
        // calls of more than 16 tokens: each size class of tiles runs gate/up, activation and
        // down on a stream of its own (the larger tiles' 64-row kernels on the caller's stream,
        // the small tiles' 16-row kernels on the side stream), joined before the combine, so
        // one class's stages fill the other's last rounds and the activation launches' idle
        // GPU. With events the stages run one after the other (each stage's two kernels at once),
        // so that each stage's times can be read.
        (void)hipEventRecord(side->fork, stream);
        (void)hipStreamWaitEvent(side->s, side->fork, 0);
        launch_mfma_class(p, 0, 2, stream);
        launch_act_class(p, 2, stream);
        launch_mfma_class(p, 1, 2, stream);
        launch_mfma_class(p, 0, 1, side->s);
        launch_act_class(p, 1, side->s);
        launch_mfma_class(p, 1, 1, side->s);
        (void)hipEventRecord(side->join, side->s);
        (void)hipStreamWaitEvent(stream, side->join, 0);
    } else if (p.mfma) {
        launch_mfma(p, 0, stream, ev(2), ev(3));
        launch_act(p, nslot, stream, ev(4), ev(5));
        launch_mfma(p, 1, stream, ev(6), ev(7));
    } else {
        // Chunks hold at most min(T, EVAMX_CHUNK) rows: each token picks an expert once, and the
        // shared expert's chunks are cut at EVAMX_CHUNK rows (repeated picks are handled in the GEMV).
        // the decode GEMV serves calls below EVAMX_MFMA_MIN_ROWS rows: one- and two-row variants
        // (a chunk with more rows, from routes that repeat an expert, runs two rows at a time)
        const int tmax = p.T <= 1 ? 1 : 2;
        {
            // one wave per item (unit, gate|up, 128 columns, k-split) over the launch's fixed
            // unit count; waves of units past the call's exit at once
            const long waves = (long)p.units_max * 2 * (p.I / 128) * ks_gate_up(p, p.units_max).base;
            const dim3 grid((unsigned)((waves + 3) / 4));
            const bool group = (p.I / 128) % ROT_WAVES == 0;
            if (route1) {
                // one more workgroup publishes the routes and records
                const dim3 grid1(grid.x + 1);
                if (group) launch_timed(moe_gate_up_route1_kernel<true>, grid1, dim3(256), stream, ev(2), ev(3), p);
                else launch_timed(moe_gate_up_route1_kernel<false>, grid1, dim3(256), stream, ev(2), ev(3), p);
            } else if (tmax == 1) {
                if (group) launch_timed(moe_gate_up_rot_kernel<1, true>, grid, dim3(256), stream, ev(2), ev(3), p);
                else launch_timed(moe_gate_up_rot_kernel<1, false>, grid, dim3(256), stream, ev(2), ev(3), p);
            } else {
                if (group) launch_timed(moe_gate_up_rot_kernel<2, true>, grid, dim3(256), stream, ev(2), ev(3), p);
                else launch_timed(moe_gate_up_rot_kernel<2, false>, grid, dim3(256), stream, ev(2), ev(3), p);
            }
        }
        launch_act(p, nslot, stream, ev(4), ev(5));
        const long waves = (long)p.units_max * (p.H / 128) * ks_down(p, p.units_max).base;
        const dim3 grid((unsigned)((waves + 3) / 4));
        if (tmax == 1) launch_timed(moe_down_rec_kernel<1>, grid, dim3(256), stream, ev(6), ev(7), p);
        else launch_timed(moe_down_rec_kernel<2>, grid, dim3(256), stream, ev(6), ev(7), p);
    }
    if (p.T <= EVAMX_SMALL_ROWS) {
        int nw = p.topk + (p.has_shared ? 1 : 0);
        if (nw > EVAMX_COMBINE_WAVES) nw = EVAMX_COMBINE_WAVES;
        if (!p.mfma)
            launch_timed(moe_combine_kernel<true>, dim3(p.T * (p.H / 128)), dim3(64 * nw), stream, ev(8), ev(9), p);
        else
            launch_timed(moe_combine_kernel<false>, dim3(p.T * (p.H / 128)), dim3(64 * nw), stream, ev(8), ev(9), p);
    } else {
        // two column groups per wave: 512 tokens 90.6 -> 88.1 us (four: 100 us, too few waves)
        if ((p.H / 128) % 2 == 0)
            launch_timed(moe_combine_rows_kernel<2>, dim3((p.T * (p.H / 256) + 3) / 4), dim3(256), stream, ev(8), ev(9), p);
        else
            launch_timed(moe_combine_rows_kernel<1>, dim3((p.T * (p.H / 128) + 3) / 4), dim3(256), stream, ev(8), ev(9), p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
