// Gate/up launches of the decode path. This unit holds the one-row launch (routing inside it);
// the multi-row kernels sit in translation units of their own (moe_gate_up2.hip, moe_gate_up8.hip,
// moe_gate_up16.hip)
// so that their instantiations compile in parallel.
#include "moe_gate_up.hpp"

namespace evamx {

void launch_gate_up_decode(const MoeParams& p, int tmax, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    // one wave per item (unit, gate|up, 128 columns, k-split) over the launch's fixed unit count;
    // waves of units past the call's exit at once
    const long waves = (long)p.units_max * 2 * (p.I / 128) * ks_gate_up(p, p.units_max).base;
    const dim3 grid((unsigned)((waves + 3) / 4));
    const bool group = (p.I / 128) % ROT_WAVES == 0;
    if (tmax == 1) {
        // one-row calls: one more workgroup publishes the routes and records
        const dim3 grid1(grid.x + 1);
        if (group) launch_timed(moe_gate_up_route1_kernel<true>, grid1, dim3(256), stream, start, stop, p);
        else launch_timed(moe_gate_up_route1_kernel<false>, grid1, dim3(256), stream, start, stop, p);
    } else if (tmax == 16 && group) {
        launch_gate_up_decode16(p, waves, stream, start, stop);
    } else if (tmax >= 8 && group) {
        launch_gate_up_decode8(p, waves, stream, start, stop);
    } else {
        launch_gate_up_decode4(p, group, grid, stream, start, stop);
    }
}

}  // namespace evamx
