// Down GEMV of the decode path (calls of 1-2 rows, and strict calls), the products on the matrix
// cores (gemv_wave_m4): one wave per (unit, 128 columns, k-split), from the unit's record. The wave
// copies its rows' activations over its k-range into its own LDS rows while its first weight loads
// are in flight, then streams the weights against them, four rows per MFMA block.
#pragma once
#include "moe_common.hpp"

namespace evamx {

constexpr int DOWN_CW = 4;                         // 128-chunks of activations per LDS window
constexpr int DOWN_RW = DOWN_CW * 64 + 8;          // words of an LDS row (padded: a quad's rows in distinct banks)
// Weight slices in flight per wave: the down items are short (32 k-slices at one token), and 3
// measured faster than 4 (one token 61.2-61.9 against 62.0-63.3 us, 16 strict tokens 422-431
// against 429-439 us, alternating runs on one box) and than 2 (down 17.6-18.3 against
// 20.5-21.0 us at one token) or 6.
constexpr int DOWN_PF = 3;

// The rows so[0..tm) of act over the 128-chunks [w0, w1) into LDS (row m at dst + m * DOWN_RW,
// chunk w0 + j at word 64 j): issue() loads them (chunks past the window reload its last one, in
// bounds and unused), finish() stores them.
template <int TM>
struct ActStage {
    static constexpr bool kWork = true;
    int tm, w0, w1, lane;
    __amdgpu_buffer_rsrc_t rs[TM];
    uint32_t* dst;
    uint32_t v[TM][DOWN_CW];

    __device__ __forceinline__ void issue()
    {
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int j = 0; j < DOWN_CW; ++j)
                v[m][j] = __builtin_amdgcn_raw_buffer_load_b32(rs[m], 4 * lane, 256 * min(w0 + j, w1 - 1), 0);
    }
    __device__ __forceinline__ void finish()
    {
#pragma unroll
        for (int m = 0; m < TM; ++m)
            if (m < tm)
#pragma unroll
                for (int j = 0; j < DOWN_CW; ++j)
                    if (w0 + j < w1) dst[m * DOWN_RW + 64 * j + lane] = v[m][j];
        wave_lds_fence();
    }
};

template <int K2, int TM>
__device__ __forceinline__ void down_rows(const MoeParams& p, const uint32_t* trellis, const int* slot, int tm, int cg,
                                             int c0, int c1, float* part, uint32_t* lds)
{
    constexpr int NG = (TM + 3) / 4;
    const int lane = threadIdx.x & 63;
    const int na = p.I / 128;
    int so[TM];
    record_slots<TM>(slot, tm, so);
    f32x4v_t acc[NG][2];
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[g][0] = acc[g][1] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
    __amdgpu_buffer_rsrc_t rs[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) rs[m] = weight_rsrc((const uint32_t*)(p.act + (size_t)so[m] * p.I));
    for (int w0 = c0; w0 < c1; w0 += DOWN_CW) {
        const int w1 = min(c1, w0 + DOWN_CW);
        if (w0 > c0) wave_lds_fence();             // the last window's reads before this one's writes
        ActStage<TM> stage{tm, w0, w1, lane, {}, lds, {}};
#pragma unroll
        for (int m = 0; m < TM; ++m) stage.rs[m] = rs[m];
        XLds4<NG> src;
        src.init(lds, DOWN_RW, 8 * w0, tm);
        gemv_wave_m4<K2, NG, DOWN_PF>(trellis, p.H / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
    }
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        if (m < tm) {
            const float xs = strided_sum<4>(p.actsum + (size_t)so[m] * na, c0, c1);   // chunk order, as gemv_chunk
            float* dst = part + (size_t)so[m] * p.H;
            dst[col0] = mul1_affine(acc[m / 4][0][m % 4], xs);
            dst[col1] = mul1_affine(acc[m / 4][1][m % 4], xs);
        }
    }
}

template <int TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void moe_down_rec_kernel(MoeParams p)
{
    __shared__ uint32_t xl[4][TMAX * DOWN_RW];
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
    uint32_t* lds = xl[threadIdx.x >> 6];
    // rows in passes of TMAX (more only when given routes repeat an expert within a token)
    for (int r0 = 0; r0 < rows; r0 += TMAX) {
        const int tr = rows - r0 < TMAX ? rows - r0 : TMAX;
        if (r0 > 0) wave_lds_fence();
        switch (k2) {
#define EVAMX_DMX(K2V) \
            case K2V: down_rows<K2V, TMAX>(p, trellis, rp->slot + r0, tr, cg, c0, c1, part, lds); break;
            EVAMX_DMX(3) EVAMX_DMX(4) EVAMX_DMX(5) EVAMX_DMX(6) EVAMX_DMX(7) EVAMX_DMX(8) EVAMX_DMX(10)
#undef EVAMX_DMX
            default: {
                // unsupported rate (flagged by the prepare): zero partials
                const int lane = threadIdx.x & 63;
                for (int m = 0; m < tr; ++m) {
                    float* dst = part + (size_t)rp->slot[r0 + m] * p.H + cg * 128;
                    dst[lane_col(lane, 0)] = 0.0f;
                    dst[lane_col(lane, 1)] = 0.0f;
                }
            }
        }
    }
}

}  // namespace evamx
