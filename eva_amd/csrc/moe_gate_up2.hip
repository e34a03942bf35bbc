// Gate/up launch of the decode path in passes of up to 2 rows (two-row calls; strict calls whose
// column groups are not a multiple of ROT_WAVES).
#include "moe_gate_up.hpp"

namespace evamx {

void launch_gate_up_decode2(const MoeParams& p, bool group, dim3 grid, hipStream_t stream, hipEvent_t start,
                            hipEvent_t stop)
{
    if (group) launch_timed(moe_gate_up_rot_kernel<2, true>, grid, dim3(256), stream, start, stop, p);
    else launch_timed(moe_gate_up_rot_kernel<2, false>, grid, dim3(256), stream, start, stop, p);
}

}  // namespace evamx
