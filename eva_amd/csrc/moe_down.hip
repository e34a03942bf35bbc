// Down GEMV of the decode path (calls of 1-2 rows, and strict calls): one wave per (unit, 128
// columns, k-split), from the unit's record, reading the activation rows through scalar loads.
#include "moe_common.hpp"

namespace evamx {

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

void launch_down_decode(const MoeParams& p, int tmax, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const long waves = (long)p.units_max * (p.H / 128) * ks_down(p, p.units_max).base;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (tmax == 1) launch_timed(moe_down_rec_kernel<1>, grid, dim3(256), stream, start, stop, p);
    else if (tmax == 2) launch_timed(moe_down_rec_kernel<2>, grid, dim3(256), stream, start, stop, p);
    else launch_timed(moe_down_rec_kernel<8>, grid, dim3(256), stream, start, stop, p);
}

}  // namespace evamx
