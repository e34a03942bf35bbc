// Down launch of the decode path for calls of 1-2 rows (and of more where the column groups are
// not a multiple of 4); the kernels sit in moe_down.hpp, the workgroup-staged kernel of strict calls
// of more than 2 rows in moe_down16.hip.
#include "moe_down.hpp"

namespace evamx {

void launch_down_decode(const MoeParams& p, int tmax, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const long waves = (long)p.units_max * (p.H / 128) * ks_down(p, p.units_max).base;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (tmax == 1) launch_timed(moe_down_rec_kernel<1>, grid, dim3(256), stream, start, stop, p);
    else if (tmax <= 4) launch_timed(moe_down_rec_kernel<4>, grid, dim3(256), stream, start, stop, p);
    else launch_timed(moe_down_rec_kernel<8>, grid, dim3(256), stream, start, stop, p);
}

}  // namespace evamx
