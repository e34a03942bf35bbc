// Gate/up launch of the decode path in passes of up to 4 rows (one MFMA row group): two-row
// calls; without the workgroup's shared LDS rows (column groups not a multiple of ROT_WAVES), every
// multi-row call, in passes of up to 2 rows.
#include "moe_gate_up.hpp"

namespace evamx {

void launch_gate_up_decode4(const MoeParams& p, bool group, dim3 grid, hipStream_t stream, hipEvent_t start,
                            hipEvent_t stop)
{
    if (group) launch_timed(moe_gate_up_rot_kernel<4, true>, grid, dim3(256), stream, start, stop, p);
    else launch_timed(moe_gate_up_rot_kernel<2, false>, grid, dim3(256), stream, start, stop, p);
}

}  // namespace evamx
