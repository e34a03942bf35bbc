// Epilogue stages of the decode-shaped MoE pipeline: the activation (gate/up partials summed in
// fixed order, SwiGLU, the down projection's input rotation) and the combine (down partials,
// output rotation, routing weights summed per token in slot order, shared expert, residual).
#include "moe_common.hpp"

namespace evamx {

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
        const SlotRec rec = load_slot_rec(p.srec + s);
        if (!rec.active) return;
        shared = rec.shared != 0;
        Sg = rec.s_gu;
        g_svh = (const half_t*)rec.g_svh;
        u_svh = (const half_t*)rec.u_svh;
        d_suh = (const half_t*)rec.d_suh;
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
void launch_act_class(const MoeParams& p, int cls, hipStream_t stream)
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
void launch_act(const MoeParams& p, int nslot, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const int na = p.I / 128;
    if (!p.mfma) {
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
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);     // uniform: the slot records load as scalars
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
            const SlotRec rec = load_slot_rec(p.srec + sk);
            if (!rec.active) {
                if (lane == 0) active[k] = 0;
                continue;
            }
            w = rec.w;
            S = rec.s_d;
            svh = (const half_t*)rec.d_svh;
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
        // the scales (and the shared expert's gate) are loaded with the partials
        const float s0 = h2f(svh[col0]), s1 = h2f(svh[col1]);
        const float gv = shared && p.sh_gate_w ? p.gate_val[row] : 1.0f;
        float v[2];
        sum_partials(p, sk, cg, lane, S, v);
        combine_item(shared, w, s0, s1, v, lane);
        if (shared && p.sh_gate_w) {
            // gated shared expert: gv * shared (exl3_moe_coop_kernel.cuh:942-948)
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
constexpr int COMBINE_BATCH = 4;      // 9 (all of DSv3's items at once) was slower: 512 tokens 88.3-88.8 -> 90.9-91.5 us

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

void launch_combine(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    if (!p.mfma || p.T <= EVAMX_SMALL_ROWS) {
        int nw = p.topk + (p.has_shared ? 1 : 0);
        if (nw > EVAMX_COMBINE_WAVES) nw = EVAMX_COMBINE_WAVES;
        if (!p.mfma)
            launch_timed(moe_combine_kernel<true>, dim3(p.T * (p.H / 128)), dim3(64 * nw), stream, start, stop, p);
        else
            launch_timed(moe_combine_kernel<false>, dim3(p.T * (p.H / 128)), dim3(64 * nw), stream, start, stop, p);
    } else {
        // two column groups per wave: 512 tokens 90.6 -> 88.1 us (four: 100 us, too few waves)
        if ((p.H / 128) % 2 == 0)
            launch_timed(moe_combine_rows_kernel<2>, dim3((p.T * (p.H / 256) + 3) / 4), dim3(256), stream, start, stop, p);
        else
            launch_timed(moe_combine_rows_kernel<1>, dim3((p.T * (p.H / 128) + 3) / 4), dim3(256), stream, start, stop, p);
    }
}

}  // namespace evamx
