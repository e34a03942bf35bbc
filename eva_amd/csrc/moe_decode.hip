// Decode-shaped cooperative EXL3 MoE layer on gfx950.
//
// Replaces the reference's prepare/rot/A/B launch sequence
// (runtime/ds41/csrc/moe_coop3072/moe_coop3072.cu:42-71) with four launches on one stream, no
// host synchronisation and no host-side memset (graph-capturable):
//
//   moe_prepare   (1 block)  routing (optional), slot activity + bounds flag, the reference
//                            run table (runs <= 8 slots, prepare_runs.cuh:8-66), per-expert
//                            chunks of <= 16 slots, counter reset
//   moe_rotate               per (slot, 128-chunk, gate|up): fp16(H128(x * suh))
//                            (exl3_moe_coop_kernel.cuh:613-629; shared expert: fp16 pre-scale,
//                            hadamard_inner.cuh:109-115)
//   moe_gemv_gu              per (chunk, gate|up, 128 columns, k-split): decode-GEMV; the last
//                            arrival per (chunk, 128 columns) runs the activation epilogue
//                            (exl3_moe_coop_kernel.cuh:758-806; shared: model.py:450-452)
//   moe_gemv_down            per (chunk, 128 columns, k-split): decode-GEMV; the last arrival
//                            per (token, 128 columns) reduces the token's slots in slot order
//                            and adds the shared expert (exl3_moe_coop_kernel.cuh:860-962,
//                            model.py:498)
#include "evamx_gemv.hpp"
#include "evamx_internal.hpp"
#include "evamx_moe.hpp"

namespace evamx {

// ---------------------------------------------------------------------------------------------
// Portable fp32 score functions (mul/add only, contraction off) so that router scores agree bit
// for bit with the CPU restatement.

#pragma clang fp contract(off)
__device__ float exp_portable(float x)
{
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float t = x * 1.4426950408889634f;
    const float n = rintf(t);
    const float r = t - n;
    float p = 1.525273380405984e-05f;
    p = p * r + 0.00015403530393381608f;
    p = p * r + 0.0013333558146428443f;
    p = p * r + 0.009618129107628477f;
    p = p * r + 0.05550410866482158f;
    p = p * r + 0.2402265069591007f;
    p = p * r + 0.6931471805599453f;
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
#pragma clang fp contract(on)

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ half_t load_x16(const void* x, int dtype, size_t i)
{
    if (dtype == EVAMX_DTYPE_F16) return ((const half_t*)x)[i];
    const uint16_t b = ((const uint16_t*)x)[i];
    return (half_t)__builtin_bit_cast(float, (uint32_t)b << 16);
}

// ---------------------------------------------------------------------------------------------
// Prepare: one block of 1024 threads.

struct PrepShared {
    int cnt[EVAMX_MAX_EXPERTS];
    int off[EVAMX_MAX_EXPERTS + 1];
    int run_base[EVAMX_MAX_EXPERTS + 1];
    int chunk_base[EVAMX_MAX_EXPERTS + 1];
    int n_active;
};

__device__ void block_exclusive_scan(int* a, int n)
{
    // In place exclusive scan of a[0..n) (n <= 1024) with a[n] = total; 1024 threads.
    const int t = threadIdx.x;
    __shared__ int buf[2][1024];
    int v = (t < n) ? a[t] : 0;
    buf[0][t] = v;
    __syncthreads();
    int src = 0;
    for (int o = 1; o < 1024; o <<= 1) {
        const int x = buf[src][t] + ((t >= o) ? buf[src][t - o] : 0);
        buf[src ^ 1][t] = x;
        src ^= 1;
        __syncthreads();
    }
    const int incl = buf[src][t];
    if (t < n) a[t] = incl - v;
    if (t == n - 1) a[n] = incl;
    if (t == 0 && n == 0) a[0] = 0;
    __syncthreads();
}

__global__ __launch_bounds__(1024) void moe_prepare_kernel(MoeParams p)
{
    __shared__ PrepShared sh;
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int slots = p.T * p.topk;
    const int E = p.n_local;

    // --- routing -------------------------------------------------------------------------
    if (p.logits) {
        for (int r = wave; r < p.T; r += 16) {
            const float* z = p.logits + (size_t)r * p.n_logits;
            float key[EVAMX_MAX_EXPERTS / 64];
            int nper = (p.n_logits + 63) / 64;
#pragma unroll
            for (int i = 0; i < EVAMX_MAX_EXPERTS / 64; ++i) {
                const int e = lane + 64 * i;
                float k = -INFINITY;
                if (i < nper && e < p.n_logits) {
                    const float zz = z[e];
                    if (p.sel_bias) k = score_fn(zz, p.score) + p.sel_bias[e];
                    else k = (p.score == EVAMX_SCORE_SIGMOID) ? zz : score_fn(zz, p.score);
                }
                key[i] = k;
            }
            float tot = 0.0f;
            float sc[EVAMX_MAX_TOPK];
            int id[EVAMX_MAX_TOPK];
            for (int j = 0; j < p.topk; ++j) {
                float bk = -INFINITY;
                int bi = 0x7fffffff;
#pragma unroll
                for (int i = 0; i < EVAMX_MAX_EXPERTS / 64; ++i) {
                    const int e = lane + 64 * i;
                    if (key[i] > bk || (key[i] == bk && e < bi)) { bk = key[i]; bi = e; }
                }
#pragma unroll
                for (int m = 1; m < 64; m <<= 1) {
                    const float ok = __shfl_xor(bk, m, WAVE);
                    const int oi = __shfl_xor(bi, m, WAVE);
                    if (ok > bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
                }
#pragma unroll
                for (int i = 0; i < EVAMX_MAX_EXPERTS / 64; ++i)
                    if (lane + 64 * i == bi) key[i] = -INFINITY;
                id[j] = bi;
                sc[j] = score_fn(z[bi], p.score);
                tot = tot + sc[j];
            }
            if (lane == 0) {
                for (int j = 0; j < p.topk; ++j) {
                    float w = sc[j] / (tot + 1e-20f);
                    w = w * p.route_scale;
                    p.sel[(size_t)r * p.topk + j] = id[j];
                    p.weights[(size_t)r * p.topk + j] = w;
                    p.rw16[(size_t)r * p.topk + j] = f2h(w);
                }
            }
        }
    } else if (p.weights) {
        for (int s = t; s < slots; s += 1024) p.rw16[s] = f2h(p.weights[s]);
    }
    if (!(p.mode & PREP_GROUP)) return;
    __syncthreads();

    // --- activity, bounds, histogram ----------------------------------------------------------
    for (int e = t; e < EVAMX_MAX_EXPERTS; e += 1024) sh.cnt[e] = 0;
    if (t == 0) sh.n_active = 0;
    __syncthreads();
    for (int s = t; s < slots; s += 1024) {
        const int64_t e = p.sel[s];
        const float w = h2f(p.rw16[s]);
        int local = -1;
        if (w != 0.0f) {
            int64_t le = e;
            bool ok = true;
            if (p.min_expert >= 0) {
                ok = e >= p.min_expert && e < p.max_expert;
                le = e - p.min_expert;
            }
            if (ok) {
                if (le < 0 || le >= E) atomicOr(p.err, EVAMX_ERR_EXPERT_RANGE);
                else local = (int)le;
            }
        }
        p.local[s] = local;
        if (local >= 0) atomicAdd(&sh.cnt[local], 1);
    }
    __syncthreads();

    // --- per-expert offsets, run bases (runs of <= 8), chunk bases (chunks of <= CHUNK) -------
    for (int e = t; e < E; e += 1024) {
        sh.off[e] = sh.cnt[e];
        sh.run_base[e] = (sh.cnt[e] + 7) / 8;
        sh.chunk_base[e] = (sh.cnt[e] + EVAMX_CHUNK - 1) / EVAMX_CHUNK;
    }
    __syncthreads();
    block_exclusive_scan(sh.off, E);
    block_exclusive_scan(sh.run_base, E);
    block_exclusive_scan(sh.chunk_base, E);
    const int n_active = sh.off[E];
    const int n_runs = sh.run_base[E];
    const int n_routed_chunks = sh.chunk_base[E];

    // --- run table (zeroed, then filled) and the sorted order ---------------------------------
    const int table_len = 2 + 2 * p.slots_max + 1;
    for (int i = t; i < table_len; i += 1024) p.runs[i] = 0;
    __syncthreads();
    int* run_start = p.runs + 2;
    int* order = p.runs + 2 + p.slots_max + 1;
    for (int s = t; s < slots; s += 1024) {
        const int e = p.local[s];
        if (e < 0) continue;
        int rank = 0;                                  // earlier active slots of the same expert
        for (int u = 0; u < s; ++u) rank += (p.local[u] == e) ? 1 : 0;
        const int pos = sh.off[e] + rank;
        order[pos] = s;
        if (p.order) p.order[pos] = s;
        if ((rank & 7) == 0) run_start[sh.run_base[e] + rank / 8] = pos;
    }
    if (t == 0) {
        p.runs[0] = n_runs;
        p.runs[1] = 0;
        run_start[n_runs] = n_active;
    }
    if (!p.order) return;                             // run table only (prepare_routes)
    // shared-expert slots follow the routed ones in the chunk order
    if (p.has_shared)
        for (int r = t; r < p.T; r += 1024) p.order[n_active + r] = slots + r;

    // --- chunks ----------------------------------------------------------------------------
    for (int e = t; e < E; e += 1024) {
        const int n = sh.cnt[e];
        for (int j = 0; j * EVAMX_CHUNK < n; ++j) {
            int* c = p.chunks + 4 * (sh.chunk_base[e] + j);
            c[0] = e;
            c[1] = sh.off[e] + j * EVAMX_CHUNK;
            c[2] = min(EVAMX_CHUNK, n - j * EVAMX_CHUNK);
            c[3] = p.k2_per_expert ? (int)p.k2_per_expert[e] : p.k2_uniform;
        }
    }
    int n_chunks = n_routed_chunks;
    if (p.has_shared) {
        const int nsc = (p.T + EVAMX_CHUNK - 1) / EVAMX_CHUNK;
        for (int j = t; j < nsc; j += 1024) {
            int* c = p.chunks + 4 * (n_routed_chunks + j);
            c[0] = -1;
            c[1] = n_active + j * EVAMX_CHUNK;
            c[2] = min(EVAMX_CHUNK, p.T - j * EVAMX_CHUNK);
            c[3] = p.k2_shared;
        }
        n_chunks += nsc;
    }
    if (t == 0) {
        p.meta[0] = n_chunks;
        p.meta[1] = n_active;
    }
    if (!(p.mode & PREP_MOE)) return;

    // --- counters, per-token arrival counts, empty rows ---------------------------------------
    for (int i = t; i < p.ctr_gu_len; i += 1024) p.ctr_gu[i] = 0;
    for (int i = t; i < p.ctr_d_len; i += 1024) p.ctr_d[i] = 0;
    __syncthreads();
    for (int r = t; r < p.T; r += 1024) {
        int n = p.has_shared ? 1 : 0;
        for (int k = 0; k < p.topk; ++k) n += (p.local[r * p.topk + k] >= 0) ? 1 : 0;
        p.tok_cnt[r] = n;
    }
    __syncthreads();
    for (int i = t; i < p.T * p.H; i += 1024) {
        const int r = i / p.H;
        if (p.tok_cnt[r] == 0) p.out[(size_t)r * p.out_stride + (i % p.H)] = 0.0f;
    }
}

// ---------------------------------------------------------------------------------------------
// Input rotation: one wave per (slot, 128-chunk, gate|up).

__global__ __launch_bounds__(256) void moe_rotate_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int item = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nch = p.H / 128;
    const int slots = p.T * p.topk;
    const int nslot = slots + (p.has_shared ? p.T : 0);
    if (item >= nslot * nch * 2) return;
    const int s = item / (nch * 2);
    const int rem = item % (nch * 2);
    const int c = rem >> 1, proj = rem & 1;
    const bool shared = s >= slots;
    int row;
    const half_t* suh;
    if (shared) {
        row = s - slots;
        suh = (const half_t*)p.sh_ptr[proj == 0 ? EVAMX_TBL_G_SUH : EVAMX_TBL_U_SUH];
    } else {
        const int e = p.local[s];
        if (e < 0) return;
        row = s / p.topk;
        suh = (const half_t*)p.tables[(size_t)(proj == 0 ? EVAMX_TBL_G_SUH : EVAMX_TBL_U_SUH) * p.tbl_stride + e];
    }
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = c * 128 + lane_col(lane, h);
        const half_t xv = load_x16(p.x, p.x_dtype, (size_t)row * p.x_stride + col);
        const half_t sv = suh[col];
        // routed: fp32 product (exl3_moe_coop_kernel.cuh:186-191); shared EXL3 linear: fp16
        // product (hadamard_inner.cuh:109-115)
        v[h] = shared ? h2f(f2h(h2f(xv) * h2f(sv))) : h2f(xv) * h2f(sv);
    }
    had128_lane(v[0], v[1], lane);
    half_t* dst = p.xr + ((size_t)proj * p.nslot_max + s) * p.H + c * 128;
    dst[lane_col(lane, 0)] = f2h(v[0]);
    dst[lane_col(lane, 1)] = f2h(v[1]);
}

__device__ __forceinline__ const void* expert_ptr(const MoeParams& p, int e, int row)
{
    if (e < 0) return (const void*)p.sh_ptr[row];
    return (const void*)p.tables[(size_t)row * p.tbl_stride + e];
}

// ---------------------------------------------------------------------------------------------
// Gate/up GEMV + activation epilogue.

__global__ __launch_bounds__(256) void moe_gemv_gu_kernel(MoeParams p, const half_t* __restrict__ xr)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.I / 128;
    const int S = p.ks_gu;
    const int c = wid / (2 * ncg * S);
    if (c >= p.meta[0]) return;
    int rem = wid % (2 * ncg * S);
    const int proj = rem / (ncg * S);
    rem %= ncg * S;
    const int cg = rem / S, ks = rem % S;

    const int* ch = p.chunks + 4 * c;
    const int e = __builtin_amdgcn_readfirstlane(ch[0]);
    const int begin = __builtin_amdgcn_readfirstlane(ch[1]);
    const int tm = __builtin_amdgcn_readfirstlane(ch[2]);
    const int k2 = __builtin_amdgcn_readfirstlane(ch[3]);
    const int* slot_of = p.order + begin;

    const int kt_n = p.H / 16;
    const int kt0 = kt_n * ks / S, kt1 = kt_n * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)expert_ptr(p, e, proj == 0 ? EVAMX_TBL_G_TRELLIS : EVAMX_TBL_U_TRELLIS);
    const half_t* A = xr + (size_t)proj * p.nslot_max * p.H;
    float* part = p.part_gu + ((size_t)ks * 2 + proj) * p.nslot_max * p.I;
    gemv_dispatch_k(k2, trellis, p.I / 16, cg, kt0, kt1, A, (size_t)p.H, slot_of, tm, part, (size_t)p.I);

    if (!arrive_last(p.ctr_gu + (size_t)c * ncg + cg, 2 * S)) return;

    // Epilogue for the chunk's slots on columns cg*128 .. +127.
    const bool shared = e < 0;
    const half_t* g_svh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_G_SVH);
    const half_t* u_svh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_U_SVH);
    const half_t* d_suh = (const half_t*)expert_ptr(p, e, EVAMX_TBL_D_SUH);
    const float L = p.limit;
    for (int m = 0; m < tm; ++m) {
        const int s = slot_of[m];
        float g[2], u[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = cg * 128 + lane_col(lane, h);
            float sg = 0.0f, su = 0.0f;
            for (int q = 0; q < S; ++q) {
                sg += p.part_gu[(((size_t)q * 2 + 0) * p.nslot_max + s) * p.I + col];
                su += p.part_gu[(((size_t)q * 2 + 1) * p.nslot_max + s) * p.I + col];
            }
            g[h] = h2f(f2h(sg));     // GEMV output stored as fp16 (gu_f32 = false)
            u[h] = h2f(f2h(su));
        }
        had128_lane(g[0], g[1], lane);
        had128_lane(u[0], u[1], lane);
        float a[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = cg * 128 + lane_col(lane, h);
            const float gs = h2f(g_svh[col]), us = h2f(u_svh[col]), ds = h2f(d_suh[col]);
            float gv, uv, x;
            if (shared) {
                // EXL3 linear outputs: fp16 after the rotation, fp16 product with svh
                gv = h2f(f2h(h2f(f2h(g[h])) * gs));
                uv = h2f(f2h(h2f(f2h(u[h])) * us));
                // swiglu: clamp the gate BEFORE SiLU (kernels.py:213-217), mid to fp16, fp16
                // product with the down projection's suh
                if (L > 0.0f) {
                    uv = fminf(fmaxf(uv, -L), L);
                    gv = fminf(gv, L);
                }
                const float mid = h2f(f2h(silu_f(gv) * uv));
                a[h] = h2f(f2h(mid * ds));
            } else {
                gv = g[h] * gs;
                uv = u[h] * us;
                x = silu_f(gv);
                if (L != 0.0f) {
                    uv = fminf(fmaxf(uv, -L), L);
                    x = fminf(x, L);
                }
                a[h] = x * uv * ds;
            }
        }
        had128_lane(a[0], a[1], lane);
        half_t* dst = p.act + (size_t)s * p.I + cg * 128;
        dst[lane_col(lane, 0)] = f2h(a[0]);
        dst[lane_col(lane, 1)] = f2h(a[1]);
    }
}

// ---------------------------------------------------------------------------------------------
// Down GEMV + per-token slot reduction.

__global__ __launch_bounds__(256) void moe_gemv_down_kernel(MoeParams p, const half_t* __restrict__ act)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.H / 128;
    const int S = p.ks_d;
    const int c = wid / (ncg * S);
    if (c >= p.meta[0]) return;
    const int rem = wid % (ncg * S);
    const int cg = rem / S, ks = rem % S;

    const int* ch = p.chunks + 4 * c;
    const int e = __builtin_amdgcn_readfirstlane(ch[0]);
    const int begin = __builtin_amdgcn_readfirstlane(ch[1]);
    const int tm = __builtin_amdgcn_readfirstlane(ch[2]);
    const int k2 = __builtin_amdgcn_readfirstlane(ch[3]);
    const int* slot_of = p.order + begin;

    const int kt_n = p.I / 16;
    const int kt0 = kt_n * ks / S, kt1 = kt_n * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)expert_ptr(p, e, EVAMX_TBL_D_TRELLIS);
    float* part = p.part_d + (size_t)ks * p.nslot_max * p.H;
    gemv_dispatch_k(k2, trellis, p.H / 16, cg, kt0, kt1, act, (size_t)p.I, slot_of, tm, part, (size_t)p.H);

    const int slots = p.T * p.topk;
    for (int m = 0; m < tm; ++m) {
        const int s = slot_of[m];
        const int row = (s < slots) ? s / p.topk : s - slots;
        if (!arrive_last(p.ctr_d + (size_t)row * ncg + cg, p.tok_cnt[row] * S)) continue;

        float o[2] = {0.0f, 0.0f};
        for (int k = 0; k < p.topk; ++k) {
            const int sk = row * p.topk + k;
            const int le = p.local[sk];
            if (le < 0) continue;
            const float w = h2f(p.rw16[sk]);
            const half_t* svh = (const half_t*)p.tables[(size_t)EVAMX_TBL_D_SVH * p.tbl_stride + le];
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = cg * 128 + lane_col(lane, h);
                float acc = 0.0f;
                for (int q = 0; q < S; ++q) acc += p.part_d[((size_t)q * p.nslot_max + sk) * p.H + col];
                v[h] = acc;
            }
            had128_lane(v[0], v[1], lane);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = cg * 128 + lane_col(lane, h);
                o[h] = o[h] + w * (v[h] * h2f(svh[col]));
            }
        }
        if (p.has_shared) {
            const int ss = slots + row;
            const half_t* svh = (const half_t*)p.sh_ptr[EVAMX_TBL_D_SVH];
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = cg * 128 + lane_col(lane, h);
                float acc = 0.0f;
                for (int q = 0; q < S; ++q) acc += p.part_d[((size_t)q * p.nslot_max + ss) * p.H + col];
                v[h] = h2f(f2h(acc));                      // EXL3 linear C in fp16
            }
            had128_lane(v[0], v[1], lane);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = cg * 128 + lane_col(lane, h);
                const float y = h2f(f2h(h2f(f2h(v[h])) * h2f(svh[col])));
                o[h] = o[h] + y;
            }
        }
        float* dst = p.out + (size_t)row * p.out_stride + cg * 128;
        dst[lane_col(lane, 0)] = o[0];
        dst[lane_col(lane, 1)] = o[1];
    }
}

// ---------------------------------------------------------------------------------------------
// Host side.

int moe_prepare_only(MoeParams& p, hipStream_t stream)
{
    hipLaunchKernelGGL(moe_prepare_kernel, dim3(1), dim3(1024), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int moe_launch(MoeParams& p, hipStream_t stream)
{
    hipLaunchKernelGGL(moe_prepare_kernel, dim3(1), dim3(1024), 0, stream, p);
    const int nch = p.H / 128;
    const int nslot = p.T * p.topk + (p.has_shared ? p.T : 0);
    {
        const int waves = nslot * nch * 2;
        hipLaunchKernelGGL(moe_rotate_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p);
    }
    {
        const int waves = p.max_chunks * 2 * (p.I / 128) * p.ks_gu;
        hipLaunchKernelGGL(moe_gemv_gu_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p, (const half_t*)p.xr);
    }
    {
        const int waves = p.max_chunks * (p.H / 128) * p.ks_d;
        hipLaunchKernelGGL(moe_gemv_down_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p, (const half_t*)p.act);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
