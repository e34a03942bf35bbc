// Down launch of strict calls of more than 2 rows. In calls of more than 8 rows each expert's 8-row
// chunks are paired as in gate/up (UnitRec::pair): the first unit's waves take both chunks' rows (up
// to 16, four MFMA row groups), so the expert's weights are decoded once for both; the second unit's
// waves exit. The
// four waves of a workgroup take four consecutive column groups of one (unit, k-split) and stage
// its activation rows into LDS once for all four (16 rows per wave would leave LDS for fewer
// waves). Every row's arithmetic is that of moe_down_rec_kernel's pass of its own chunk.
#include "moe_down.hpp"

namespace evamx {

constexpr int DOWN_GROUP_WAVES = 4;
static_assert(DOWN_GROUP_WAVES == DOWN_CW, "each wave stages one chunk of a window");
// Weight slices in flight per wave in 16-row passes (four row groups' accumulators and activations
// leave fewer registers for the ring).
constexpr int DOWN_PAIR_PF = 3;

// The rows so[0..TM) of act over the 128-chunks [w0, w1), staged once for the workgroup: wave w
// copies chunk w0 + w of every row (rows past tm copy row so[0], in bounds and unused; a wave past
// the window copies nothing), then the workgroup meets at a barrier.
template <int TM>
struct ActStageGroup {
    static constexpr bool kWork = true;
    int tm, w0, w1, lane, wave;
    __amdgpu_buffer_rsrc_t rs;                    // the activation rows' base
    const uint32_t (&roff)[TM];                   // byte offset of each row
    uint32_t* dst;
    uint32_t v[TM];

    __device__ __forceinline__ void issue()
    {
        const int c = min(w0 + wave, w1 - 1);
#pragma unroll
        for (int m = 0; m < TM; ++m) v[m] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * lane, roff[m] + 256 * c, 0);
    }
    __device__ __forceinline__ void finish()
    {
        if (w0 + wave < w1) {
#pragma unroll
            for (int m = 0; m < TM; ++m)
                if (m < tm) dst[m * DOWN_RW + 64 * wave + lane] = v[m];
        }
        __syncthreads();
    }
};

template <int K2, int TM>
__device__ __forceinline__ void down_rows_group(const MoeParams& p, const uint32_t* trellis, const int (&so)[TM], int tm,
                                                int cg, int c0, int c1, float* part, uint32_t* lds)
{
    constexpr int NG = (TM + 3) / 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int na = p.I / 128;
    f32x4v_t acc[NG][2];
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[g][0] = acc[g][1] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t roff[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) roff[m] = __builtin_amdgcn_readfirstlane((uint32_t)so[m] * (uint32_t)p.I * 2u);
    const __amdgpu_buffer_rsrc_t rs = weight_rsrc((const uint32_t*)p.act);
    for (int w0 = c0; w0 < c1; w0 += DOWN_CW) {
        const int w1 = min(c1, w0 + DOWN_CW);
        if (w0 > c0) __syncthreads();             // every wave's reads of the last window before this one's writes
        ActStageGroup<TM> stage{tm, w0, w1, lane, wave, rs, roff, lds, {}};
        XLds4<NG> src;
        src.init(lds, DOWN_RW, 8 * w0, tm);
        gemv_wave_m4<K2, NG, (TM > 8 ? DOWN_PAIR_PF : DOWN_PF)>(trellis, p.H / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
    }
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        if (m < tm) {
            const float xs = strided_sum<4>(p.actsum + (size_t)so[m] * na, c0, c1);   // chunk order, as down_rows
            float* dst = part + (size_t)so[m] * p.H;
            dst[col0] = mul1_affine(acc[m / 4][0][m % 4], xs);
            dst[col1] = mul1_affine(acc[m / 4][1][m % 4], xs);
        }
    }
}

template <int K2>
__device__ __forceinline__ void down_pair(const MoeParams& p, const uint32_t* trellis, const UnitRec* rp, int rows,
                                          int rows_b, int cg, int c0, int c1, float* part, uint32_t* lds)
{
    if (rows_b == 0) {
        int so[8];
        record_slots<8>(rp->slot, rows, so);
        down_rows_group<K2, 8>(p, trellis, so, rows, cg, c0, c1, part, lds);
        return;
    }
    int so[16];                                   // the first unit is a full chunk
    record_slots<8>(rp->slot, 8, *(int(*)[8])so);
    record_slots<8>(rp[1].slot, rows_b, *(int(*)[8])(so + 8));
    down_rows_group<K2, 16>(p, trellis, so, 8 + rows_b, cg, c0, c1, part, lds);
}

// One wave per (unit, k-split, 128 columns), column groups fastest (the column groups a multiple
// of DOWN_GROUP_WAVES, so a workgroup never spans two (unit, k-split) items).
__global__ __launch_bounds__(64 * DOWN_GROUP_WAVES) __attribute__((amdgpu_waves_per_eu(4))) void moe_down_pair_kernel(MoeParams p)
{
    __shared__ uint32_t xl[16 * DOWN_RW];
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.H / 128;
    const KSplit k = ks_down(p, p.units_max);
    const int per_unit = ncg * k.base;
    const int u = __builtin_amdgcn_readfirstlane(wid / per_unit);
    if (u >= p.units_max) return;
    const UnitRec* rp = p.urec + u;
    const int e = __builtin_amdgcn_readfirstlane(rp->e);
    if (e == EVAMX_NO_UNIT) return;
    const int pair = __builtin_amdgcn_readfirstlane(rp->pair);
    if (pair < 0) return;                         // the previous unit's waves take these rows
    const int ubase = __builtin_amdgcn_readfirstlane(rp->ubase);
    const int S = __builtin_amdgcn_readfirstlane(rp->s_d);
    const int r = wid - ubase * per_unit;
    if (r >= ncg * S) return;
    const int cg = __builtin_amdgcn_readfirstlane(r % ncg), ks = __builtin_amdgcn_readfirstlane(r / ncg);
    const int rows = __builtin_amdgcn_readfirstlane(rp->rows);
    const int rows_b = pair > 0 ? __builtin_amdgcn_readfirstlane(rp[1].rows) : 0;
    const int k2 = __builtin_amdgcn_readfirstlane(rp->k2_d);
    const int na = p.I / 128;
    const int c0 = na * ks / S, c1 = na * (ks + 1) / S;
    const uint32_t* trellis = (const uint32_t*)rp->tr[2];
    float* part = p.part_d + (size_t)ks * moe_nslot(p) * p.H;
    switch (k2) {
#define EVAMX_DPX(K2V) \
        case K2V: down_pair<K2V>(p, trellis, rp, rows, rows_b, cg, c0, c1, part, xl); break;
        EVAMX_DPX(3) EVAMX_DPX(4) EVAMX_DPX(5) EVAMX_DPX(6) EVAMX_DPX(7) EVAMX_DPX(8) EVAMX_DPX(10)
#undef EVAMX_DPX
        default: {
            // unsupported rate (flagged by the prepare): zero partials
            const int lane = threadIdx.x & 63;
            for (int h = 0; h < (rows_b > 0 ? 2 : 1); ++h)
                for (int m = 0; m < (h ? rows_b : rows); ++m) {
                    float* dst = part + (size_t)rp[h].slot[m] * p.H + cg * 128;
                    dst[lane_col(lane, 0)] = 0.0f;
                    dst[lane_col(lane, 1)] = 0.0f;
                }
        }
    }
}

void launch_down_decode16(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const long waves = (long)p.units_max * (p.H / 128) * ks_down(p, p.units_max).base;
    const dim3 grid((unsigned)((waves + DOWN_GROUP_WAVES - 1) / DOWN_GROUP_WAVES));
    launch_timed(moe_down_pair_kernel, grid, dim3(64 * DOWN_GROUP_WAVES), stream, start, stop, p);
}

}  // namespace evamx
