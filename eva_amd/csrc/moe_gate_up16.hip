// Gate/up launch of the decode path for strict calls of more than 8 rows: an expert's chunks
// paired, up to 16 rows per pass (the column groups a multiple of ROT_WAVES), in a translation
// unit of its own so that its instantiations compile in parallel with the others.
#include "moe_gate_up.hpp"

namespace evamx {

void launch_gate_up_decode16(const MoeParams& p, long waves, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    // eight column groups per workgroup where they divide the column groups: each workgroup's
    // rows are rotated once for eight column groups instead of four
    if ((p.I / 128) % 8 == 0)
        launch_timed(moe_gate_up_rot_kernel<16, true, 8>, dim3((unsigned)((waves + 7) / 8)), dim3(512), stream, start, stop, p);
    else
        launch_timed(moe_gate_up_rot_kernel<16, true, 4>, dim3((unsigned)((waves + 3) / 4)), dim3(256), stream, start, stop, p);
}

}  // namespace evamx
