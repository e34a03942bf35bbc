// Decode-shaped cooperative EXL3 MoE layer on gfx950.
//
// Replaces the reference's prepare/rot/A/B launch sequence
// (runtime/ds41/csrc/moe_coop3072/moe_coop3072.cu:42-71). Cross-workgroup results only ever
// cross a kernel boundary: a device-scope release fence costs an L2 write-back on this
// multi-XCD part, far more than a launch when thousands of waves would each need one. Five
// stages on one stream, no host synchronisation, no memset (graph-capturable):
//
//   (gate)        optional router front: fp32 logits x . gate_w (model.py:404-409)
//   moe_prepare   routing (optional), slot activity + bounds flag, stable grouping by expert
//                 (the reference run table, runs <= 8 slots: prepare_runs.cuh:8-66; and chunks
//                 of <= 8 slots for the GEMV work items, or tiles of <= 64 for the MFMA path),
//                 then the input rotation fp16(H128(x * suh)) of every active slot
//                 (exl3_moe_coop_kernel.cuh:613-629; shared expert: fp16 pre-scale,
//                 hadamard_inner.cuh:109-115). For 3-16 rows one kernel: every workgroup
//                 routes, workgroup 0 groups and publishes the tables, the others rotate.
//                 Decode path (1-2 rows): unit and slot records instead of tables, no rotation
//                 launch (the gate/up waves rotate their own inputs); 2 rows: one workgroup;
//                 1 row: no prepare launch (the gate/up launch routes).
//   moe_gate_up   per (unit, gate|up, 128 columns, k-split) wave: decode GEMV -> fp32 partials
//                 (3 rows and more: MFMA tiles, moe_prefill.hip)
//   moe_act       per (active slot, 128 columns of I): sums the gate/up partials in fixed
//                 order, rounds to fp16 (gu_f32 = false), and runs the activation epilogue
//                 (exl3_moe_coop_kernel.cuh:758-806; shared expert: model.py:450-452)
//   moe_down      per (chunk, 128 columns, k-split) wave: decode GEMV -> fp32 partials
//                 (3 rows and more: MFMA tiles)
//   moe_combine   per (token, 128 columns): output rotation * svh * routing weight, summed over
//                 the token's slots in slot order, plus the shared expert
//                 (exl3_moe_coop_kernel.cuh:860-962, model.py:498)
#include <cstdlib>
#include <cstring>
#include "evamx_gemv.hpp"
#include "evamx_internal.hpp"
#include "evamx_moe.hpp"
namespace evamx {

int moe_launch(MoeParams& p, hipStream_t stream, void* const* events)
{
    // events[2k] / events[2k + 1]: start of the first and end of the last kernel of stage k
    auto ev = [&](int i) { return events ? (hipEvent_t)events[i] : (hipEvent_t) nullptr; };
    const int nslot = p.T * p.topk + (p.has_shared ? p.T : 0);
    // strict mode: a call of up to strict_rows rows runs the decode path with the one-row k-splits
    // (given as requested splits, so every chunk takes them whatever its rows), so every row is
    // computed as it would be alone
    p.strict = p.strict_rows > 0 && p.T <= p.strict_rows ? 1 : 0;
    if (p.strict) {
        p.ks_gu = p.strict_ks_gu;
        p.ks_d = p.strict_ks_d;
    }
    p.mfma = !p.strict && p.T >= EVAMX_MFMA_MIN_ROWS ? 1 : 0;
    // up to 16 tokens only the 16-row MFMA kernel runs, so the tiles are cut at 16 rows (more
    // than 16 slots of one expert occur only when given routes repeat an expert within a token)
    p.chunk_rows = !p.mfma ? EVAMX_CHUNK : p.T <= EVAMX_SMALL_TILE_ROWS ? EVAMX_SMALL_TILE_ROWS : EVAMX_TILE_ROWS;
    // decode path: chunks of at most 8 rows weigh at most their row count, so the call has at
    // most one unit per slot plus the shared expert's chunks
    p.units_max = moe_units_max(p.T, p.topk, p.has_shared);
    hipEvent_t first = ev(0);
    // one-row calls route inside the gate/up launch: their prepare stage is the router front
    // alone (given gate_w), else it has no kernel and records no events
    const bool route1 = !p.mfma && p.T == 1;
    if (p.gate_w) {
        launch_router_front(p, stream, first, route1 ? ev(1) : nullptr);
        first = nullptr;
    }
    if (!route1) launch_prepare(p, stream, first, ev(1));
    const SideStream* side = p.mfma && p.T > EVAMX_SMALL_TILE_ROWS && p.side_ok && !events ? side_stream(stream) : nullptr;
    if (side) {
        // calls of more than 16 tokens: each size class of tiles runs gate/up, activation and
        // down on a stream of its own (the larger tiles' 64-row kernels on the caller's stream,
        // the small tiles' 16-row kernels on the side stream), joined before the combine, so
        // one class's stages fill the other's last rounds and the activation launches' idle
        // GPU. With events the stages run one after the other (each stage's two kernels at once),
        // so that each stage's times can be read.
        (void)hipEventRecord(side->fork, stream);
        (void)hipStreamWaitEvent(side->s, side->fork, 0);
        launch_mfma_class(p, 0, 2, stream);
        launch_act_class(p, 2, stream);
        launch_mfma_class(p, 1, 2, stream);
        launch_mfma_class(p, 0, 1, side->s);
        launch_act_class(p, 1, side->s);
        launch_mfma_class(p, 1, 1, side->s);
        (void)hipEventRecord(side->join, side->s);
        (void)hipStreamWaitEvent(stream, side->join, 0);
    } else if (p.mfma) {
        launch_mfma(p, 0, stream, ev(2), ev(3));
        launch_act(p, nslot, stream, ev(4), ev(5));
        launch_mfma(p, 1, stream, ev(6), ev(7));
    } else {
        // The decode GEMV serves calls below EVAMX_MFMA_MIN_ROWS rows and strict calls. Chunks
        // hold at most min(T, EVAMX_CHUNK) rows (each token picks an expert once; the shared
        // expert's chunks are cut at EVAMX_CHUNK rows); the kernels run one-, two- or eight-row
        // passes, and a chunk with more rows than the pass (given routes that repeat an expert)
        // runs in several.
        const int tmax = p.T <= 1 ? 1 : p.T <= 2 ? 2 : 8;
        // strict calls of more than 8 rows: gate/up and down take an expert's chunks in pairs
        // (its weights decoded once for up to 16 rows). Strict down of more than 2 rows runs the
        // workgroup-staged kernel with or without pairs (58 layers at 8 tokens and 2.5 bpw: 20.50-20.60
        // against 20.88-20.95 ms; one 8-token layer at 4 bpw 1.5% slower).
        const bool pairs = pair_units(p);
        launch_gate_up_decode(p, pairs ? 16 : tmax, stream, ev(2), ev(3));
        launch_act(p, nslot, stream, ev(4), ev(5));
        if (pairs || (p.strict && p.T > 2 && (p.H / 128) % 4 == 0)) launch_down_decode16(p, stream, ev(6), ev(7));
        else launch_down_decode(p, tmax, stream, ev(6), ev(7));
    }
    launch_combine(p, stream, ev(8), ev(9));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
