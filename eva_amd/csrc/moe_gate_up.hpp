// Gate/up GEMV kernels of the decode path (calls of 1-2 rows, and strict calls): each wave
// rotates its own inputs into LDS and streams its weights, the products on the matrix cores
// (moe_gate_up.hip instantiates the one-row kernel, moe_gate_up2.hip the 2- and 4-row ones,
// moe_gate_up8.hip the 8-row one, moe_gate_up16.hip the one of paired 8-row chunks).
#pragma once
#include "moe_common.hpp"

namespace evamx {

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

// The same rotations shared by the NW waves of a workgroup (four, or eight in the strict kernels),
// which then stream NW column groups of the same (unit, projection, k-split): wave w rotates chunks
// w, w + NW, ... of the window (CW chunks at most) into the workgroup's LDS rows and stores each
// chunk's sum. After a
// barrier the rows are ready; add_sums() adds a row's chunk sums in chunk order (the order of the
// per-wave stage, so the results are the same), after the GEMV so that the sums hold no
// registers during it. The rows' x words load through one resource with per-row scalar offsets.
constexpr int ROT_WAVES = 4;

template <int TM, int NW = ROT_WAVES, int CW = ROT_CW>
struct RotStageGroup {
    static constexpr bool kWork = true;
    static constexpr int NJ = CW / NW;                 // chunks per wave and window
    static_assert(CW % NW == 0, "a window's chunks split evenly over the waves");
    const MoeParams& p;
    const int (&so)[TM];
    int tm, w0, w1, row_words, lane, wave;
    __amdgpu_buffer_rsrc_t suh_rsrc, x_rsrc;           // suh of the projection; x from row 0
    const uint32_t (&xoff)[TM];                         // byte offset of each row's x
    uint32_t* dst;                                      // LDS rows
    float* sums;                                        // LDS [TM][CW] chunk sums
    uint32_t xv[TM][NJ], sv[NJ];

    __device__ __forceinline__ int chunk(int i) const { return min(w0 + wave + NW * i, w1 - 1); }
    __device__ __forceinline__ void issue()
    {
#pragma unroll
        for (int i = 0; i < NJ; ++i) sv[i] = __builtin_amdgcn_raw_buffer_load_b32(suh_rsrc, 4 * lane, 256 * chunk(i), 0);
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int i = 0; i < NJ; ++i)
                xv[m][i] = __builtin_amdgcn_raw_buffer_load_b32(x_rsrc, 4 * lane, xoff[m] + 256 * chunk(i), 0);
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
                    if (lane == 0) sums[m * CW + (c - w0)] = sm;
                }
            }
        }
        __syncthreads();
    }
};

template <int TM, int CW>
__device__ __forceinline__ void add_sums(const float* sums, int tm, int nc, float (&xs)[TM])
{
#pragma unroll
    for (int m = 0; m < TM; ++m)
        if (m < tm)
            for (int c = 0; c < nc; ++c) xs[m] += sums[m * CW + c];
}

// Chunks of rotated input per LDS window and row of a kernel whose passes take up to TM rows:
// ROT_CW, and 8 for 16-row passes (a strict call's k-splits span 8 chunks at the DSv3 shape), so
// that 16 rows take the LDS of 8 rows of ROT_CW chunks.
template <int TM>
constexpr int rot_cw() { return TM > 8 ? 8 : ROT_CW; }

// Weight slices in flight per wave in 16-row passes (the four row groups' accumulators and
// activations leave fewer registers for the ring).
constexpr int PAIR_PF = 3;

// Words of an LDS row of rotated inputs: CW chunks, padded so that the four rows a lane quad
// reads start in different banks.
template <int CW>
constexpr int rot_row_words() { return CW * 64 + 8; }
constexpr int ROT_ROW_WORDS = rot_row_words<ROT_CW>();

// Gate/up GEMV of tm rows (slots slot[0..tm)) over the 128-chunks [c0, c1): each window of at
// most rot_cw<TM>() chunks is rotated into LDS (GROUP: by the workgroup's NW waves together),
// then streamed with the products on the matrix cores (gemv_wave_m4, rows in groups of four);
// writes the fp32 partials of the rows.
template <int K2, int TM, bool GROUP, int NW = ROT_WAVES>
__device__ __forceinline__ void gate_up_rot_rows(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                 const int (&so)[TM], int tm, int cg, int c0, int c1, float* part,
                                                 uint32_t* lds, float* lsums)
{
    const int lane = threadIdx.x & 63;
    constexpr int NG = (TM + 3) / 4;
    constexpr int CW = rot_cw<TM>();
    f32x4v_t acc[NG][2];
    float xs[TM];
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[g][0] = acc[g][1] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < TM; ++m) xs[m] = 0.0f;
    constexpr int RW = rot_row_words<CW>();
    const int slots = p.T * p.topk;
    const __amdgpu_buffer_rsrc_t srs = weight_rsrc((const uint32_t*)suh);
    auto window = [&](int w0, int w1) __attribute__((always_inline)) {
        XLds4<NG> src;
        src.init(lds, RW, 8 * w0, tm);
        if constexpr (GROUP) {
            // the wave index made provably uniform: the chunk offsets of the staging loads are then scalar
            // (a per-lane offset puts every load in a loop over the distinct offsets)
            const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
            uint32_t xoff[TM];
#pragma unroll
            for (int m = 0; m < TM; ++m) {
                const int row = so[m] >= slots ? so[m] - slots : so[m] / p.topk;
                xoff[m] = __builtin_amdgcn_readfirstlane((uint32_t)row * (uint32_t)p.x_stride * 2u);
            }
            RotStageGroup<TM, NW, CW> stage{p, so, tm, w0, w1, RW, lane, wave, srs, weight_rsrc((const uint32_t*)p.x), xoff,
                                            lds, lsums, {}, {}};
            gemv_wave_m4<K2, NG, NG == 4 ? PAIR_PF : 4>(trellis, p.I / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
            add_sums<TM, CW>(lsums, tm, w1 - w0, xs);
        } else {
            RotStage<TM> stage{p, so, tm, w0, w1, RW, lane, srs, {}, lds, xs};
#pragma unroll
            for (int m = 0; m < TM; ++m) {
                const int row = so[m] >= slots ? so[m] - slots : so[m] / p.topk;
                stage.x_rsrc[m] = weight_rsrc((const uint32_t*)((const uint16_t*)p.x + (size_t)row * p.x_stride));
            }
            gemv_wave_m4<K2, NG>(trellis, p.I / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
        }
    };
    if (c1 - c0 <= CW) {
        window(c0, c1);                 // the common case, straight-line
    } else {
        for (int w0 = c0; w0 < c1; w0 += CW) {
            window(w0, min(c1, w0 + CW));
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
            dst[col0] = mul1_affine(acc[m / 4][0][m % 4], xs[m]);
            dst[col1] = mul1_affine(acc[m / 4][1][m % 4], xs[m]);
        }
    }
}

// tm rows (at most TMAX; slots slot[0..tm) of a unit record) through one TMAX-row variant per rate
// (rows past tm are skipped): the kernel's register budget is its widest variant's anyway, every
// smaller variant as well would make its compile several times longer, and every row's arithmetic
// is the same whatever the variant (rows are independent accumulators).
template <int K2, int TMAX, bool GROUP, int NW = ROT_WAVES>
__device__ __forceinline__ void gate_up_rot_fit(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                const int* slot, int tm, int cg, int c0, int c1, float* part,
                                                uint32_t* lds, float* lsums)
{
    static_assert(TMAX == 1 || TMAX == 2 || TMAX == 4 || TMAX == 8, "decode path rows: 1, 2, 4 or 8 per unit pass");
    int so[TMAX];
    record_slots<TMAX>(slot, tm, so);
    gate_up_rot_rows<K2, TMAX, GROUP, NW>(p, trellis, suh, so, tm, cg, c0, c1, part, lds, lsums);
}

template <int K2, int TMAX, bool GROUP, int NW = ROT_WAVES>
__device__ __forceinline__ void gate_up_rot_item(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                 const int* slot, int rows, int cg, int c0, int c1, float* part,
                                                 uint32_t* lds, float* lsums)
{
    // one pass in the common case; a chunk of more than TMAX rows (given routes that repeat an
    // expert, or 8-row chunks in the 2-row kernel) runs TMAX rows at a time (one call site, so
    // the GEMV is inlined once)
    for (int r0 = 0;; r0 += TMAX) {
        const int tr = rows - r0 < TMAX ? rows - r0 : TMAX;
        gate_up_rot_fit<K2, TMAX, GROUP, NW>(p, trellis, suh, slot + r0, tr, cg, c0, c1, part, lds, lsums);
        if (r0 + TMAX >= rows) break;
        if constexpr (GROUP) __syncthreads();      // this pass's LDS reads before the next pass's writes
        else wave_lds_fence();
    }
}

// Paired units (TMAX 16, strict calls): a unit whose record says pair > 0 takes its own rows and
// the next unit's (two chunks of one expert, at most 16 rows) in one pass, so the expert's weights
// are decoded once for both; the next unit's waves exit. Every row's arithmetic is that of a pass
// of its own chunk.
template <int K2, bool GROUP, int NW>
__device__ __forceinline__ void gate_up_rot_pair(const MoeParams& p, const uint32_t* trellis, const half_t* suh,
                                                 const UnitRec* rp, int rows, int rows_b, int cg, int c0, int c1,
                                                 float* part, uint32_t* lds, float* lsums)
{
    if (rows_b == 0) {
        // a unit alone: the 8-row kernel's pass
        int so[8];
        record_slots<8>(rp->slot, rows, so);
        gate_up_rot_rows<K2, 8, GROUP, NW>(p, trellis, suh, so, rows, cg, c0, c1, part, lds, lsums);
        return;
    }
    int so[16];                                   // the first unit is a full chunk
    record_slots<8>(rp->slot, 8, *(int(*)[8])so);
    record_slots<8>(rp[1].slot, rows_b, *(int(*)[8])(so + 8));
    gate_up_rot_rows<K2, 16, GROUP, NW>(p, trellis, suh, so, 8 + rows_b, cg, c0, c1, part, lds, lsums);
}

// One wave per (unit, gate|up, k-split, 128 columns), NWG waves per workgroup. GROUP (the
// column-group count a multiple of NWG): the items run column group fastest, so the waves of a
// workgroup share unit, projection and k-split (and exit together) and rotate their inputs
// together; otherwise every wave rotates its own (four waves per workgroup).
template <int TMAX, bool GROUP, int NWG = ROT_WAVES>
__global__ __launch_bounds__(64 * NWG) __attribute__((amdgpu_waves_per_eu(4))) void moe_gate_up_rot_kernel(MoeParams p)
{
    static_assert(GROUP || NWG == 4, "waves that rotate their own rows run four to a workgroup");
    static_assert(TMAX != 16 || GROUP, "paired units run with the workgroup's shared rows");
    __shared__ uint32_t xl[GROUP ? 1 : NWG][TMAX * rot_row_words<rot_cw<TMAX>()>()];
    __shared__ float xsums[TMAX * rot_cw<TMAX>()];
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
    int rows_b = 0;                             // rows of the paired next unit
    if constexpr (TMAX == 16) {
        const int pair = __builtin_amdgcn_readfirstlane(rp->pair);
        if (pair < 0) return;                   // the previous unit's waves take these rows
        if (pair > 0) rows_b = __builtin_amdgcn_readfirstlane(rp[1].rows);
    }
    const int k2 = __builtin_amdgcn_readfirstlane(rp->k2);
    const int nch = p.H / 128;
    const int c0 = nch * ks / S, c1 = nch * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)rp->tr[proj];
    const half_t* suh = (const half_t*)rp->suh[proj];
    float* part = p.part_gu + ((size_t)ks * 2 + proj) * moe_nslot(p) * p.I;
    uint32_t* lds = xl[GROUP ? 0 : wave];
    switch (k2) {
#define EVAMX_GUX(K2V)                                                                                       \
        case K2V:                                                                                            \
            if constexpr (TMAX == 16)                                                                        \
                gate_up_rot_pair<K2V, GROUP, NWG>(p, trellis, suh, rp, rows, rows_b, cg, c0, c1, part, lds, xsums); \
            else                                                                                             \
                gate_up_rot_item<K2V, TMAX, GROUP, NWG>(p, trellis, suh, rp->slot, rows, cg, c0, c1, part, lds, xsums); \
            break;
        EVAMX_GUX(3) EVAMX_GUX(4) EVAMX_GUX(5) EVAMX_GUX(6) EVAMX_GUX(7) EVAMX_GUX(8) EVAMX_GUX(10)
#undef EVAMX_GUX
        default: {
            // unsupported rate (flagged by the prepare): zero partials, so no output reads stale data
            const int lane = threadIdx.x & 63;
            for (int h = 0; h < (rows_b > 0 ? 2 : 1); ++h)
                for (int m = 0; m < (h ? rows_b : rows); ++m) {
                    float* dst = part + (size_t)rp[h].slot[m] * p.I + cg * 128;
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
    __shared__ uint32_t xl[GROUP ? 1 : 4][ROT_ROW_WORDS];
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
        auto route = [&]() {
            int id;
            half_t rw;
            float w32;
            slot_routes1(p, lane, id, rw, w32);
            id = __builtin_amdgcn_readlane(id, u);
            const half_t rwu = __builtin_bit_cast(half_t, (uint16_t)__builtin_amdgcn_readlane((int)__builtin_bit_cast(uint16_t, rw), u));
            return __builtin_amdgcn_readfirstlane(slot_local(p, id, rwu, false));
        };
        if constexpr (GROUP) {
            // the workgroup's four waves share the slot: one routes, the others wait for it
            __shared__ int e_sh;
            if (wave == 0) {
                const int e0 = route();
                if (lane == 0) e_sh = e0;
            }
            __syncthreads();
            e = __builtin_amdgcn_readfirstlane(e_sh);
        } else {
            e = route();
        }
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

}  // namespace evamx
