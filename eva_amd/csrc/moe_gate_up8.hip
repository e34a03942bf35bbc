// Gate/up launch of the decode path with chunks of up to 8 rows (strict calls of 3 or more
// rows; the column groups a multiple of ROT_WAVES), in a translation unit of its own so that its
// instantiations compile in parallel with the others.
#include "moe_gate_up.hpp"

namespace evamx {

void launch_gate_up_decode8(const MoeParams& p, long waves, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    // eight column groups per workgroup where they divide the column groups: each workgroup's
    // rows are rotated once for eight column groups instead of four
    if ((p.I / 128) % 8 == 0)
        launch_timed(moe_gate_up_rot_kernel<8, true, 8>, dim3((unsigned)((waves + 7) / 8)), dim3(512), stream, start, stop, p);
    else
        launch_timed(moe_gate_up_rot_kernel<8, true, 4>, dim3((unsigned)((waves + 3) / 4)), dim3(256), stream, start, stop, p);
}

}  // namespace evamx
