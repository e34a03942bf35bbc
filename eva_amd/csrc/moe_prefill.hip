// Prefill-shaped expert GEMMs on gfx950: trellis decode into LDS feeding fp16 MFMA.
//
// Replaces the reference's grouped expert matmuls for large batches (the coop kernels'
// gemv_tile, exl3_moe_coop_kernel.cuh:340-544, run once per <= 8-row run). Here a work item is
// (tile of <= 64 grouped rows of one expert, 128 output columns, projection), one wave each,
// over the full k range, so every weight is decoded once per 64 rows instead of once per 8:
//
//   - the wave streams its 8 trellis tiles per k-slice exactly like the decode GEMV (lane
//     8*i + q owns tile i's columns q, q + 8) and decodes two k-slices into the (1024 +
//     bytesum) fp16 values of the affine codebook map (w = 0x1eee * h + 0xc931);
//   - it restages them through a wave-private 8 KiB LDS region into the B operands of
//     v_mfma_f32_16x16x32_f16 (lane n + 16 g holds column n, k = 8g .. 8g+7), one per 16-column
//     tile, and reads the rotated activations of its rows as the A operands (lane m + 16 g
//     holds row m, the same k) straight from global memory;
//   - 4 x 8 accumulators (64 rows x 128 columns, fp32) take sum_k x_k h_k, and the epilogue
//     applies the codebook map per column with the rows' activation sums, as the decode GEMV
//     does, writing the same fp32 partials (one k-split).
//
// The LDS exchange stays within a wave (a wave's LDS instructions execute in order), so the
// waves of a workgroup never synchronise.
//
// Calls of more than 16 tokens run two kernels per stage: the tiles of at most 16 rows in the
// 16-row kernel (a quarter of the accumulators, 4 waves per SIMD) on the calling thread's side
// stream, the larger ones in the 64-row kernel (2 waves per SIMD) on the caller's stream, at the
// same time; moe_launch pipelines each size class through gate/up, activation and down on its
// stream (launch_mfma_class), launch_mfma runs one stage's two kernels at once.

#include <stdlib.h>
#include <string.h>

#include "evamx_internal.hpp"
#include "evamx_mfma.hpp"
#include "evamx_moe.hpp"

namespace evamx {

constexpr int MF_WAVES = 4;                     // waves per workgroup

template <int K2, int MBMAX>
__device__ __forceinline__ void mfma_item_rows(const uint32_t* trellis, int nt_n, int cg, int kt0, int kt1,
                                               const GlobalRows& src, const int* slot_of, int rows, float* part,
                                               size_t part_stride, uint32_t* lds)
{
    // both kernels run their items with progress priorities: the 16-row kernel's equal items,
    // and the 64-row kernel's items of 1-4 row blocks since they share the GPU with the 16-row
    // kernel on another stream (512 tokens: gate/up 1319-1331 -> 1268-1287 us)
    if constexpr (MBMAX == 1) {
        mfma_item<K2, 1, true>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, lds);
    } else {
        const int mb = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
        switch (mb) {
            case 1: mfma_item<K2, 1, true>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, lds); break;
            case 2: mfma_item<K2, 2, true>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, lds); break;
            case 3: mfma_item<K2, 3, true>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, lds); break;
            default: mfma_item<K2, 4, true>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, lds); break;
        }
    }
}

// Workgroup -> item block with the items of one tile on one XCD: workgroups are dispatched to
// the 8 XCDs round robin, so consecutive item blocks (a tile's column groups, which share its
// activation rows) are given to workgroups b, b + 8, b + 16, ... (nb a multiple of 8).
__device__ __forceinline__ int xcd_item_block(int b, int nb)
{
    const int per = nb >> 3;
    if ((nb & 7) != 0 || per == 0) return b;
    return (b & 7) * per + (b >> 3);
}

// which = 0: gate/up, items (tile, proj, cg, ks) with cg over I/128 -> part_gu[ks][proj][slot][I];
// which = 1: down, items (tile, cg, ks) with cg over H/128 -> part_d[ks][slot][H].
// Every tile is one work unit of weight 1; the k-split is the decode GEMV's (moe_ksplit: as many
// splits as fill the resident grid once, or the requested count), so the activation and combine
// kernels sum the same partials. MBMAX bounds the tile rows in 16-row blocks: the MBMAX 1 kernel
// (a quarter of the accumulators, 4 waves per SIMD) runs the tiles of at most 16 rows, the
// MBMAX 4 kernel the larger ones; the split count is the same for both (from all the tiles).
template <int MBMAX, int which>
__device__ __forceinline__ void mfma_stage(const MoeParams& p, uint32_t (&lds)[MF_WAVES][MF_LDS_WORDS])
{
    const int wave = threadIdx.x >> 6;
    const int n_all = __builtin_amdgcn_readfirstlane(p.meta[0]);
    const int n_small = __builtin_amdgcn_readfirstlane(p.meta[3]);
    const int ncg = which == 0 ? p.I / 128 : p.H / 128;
    const KSplit k = which == 0 ? ks_gate_up(p, n_all) : ks_down(p, n_all);
    const int S = ks_of_chunk(k, 1);
    const int per_tile = (which == 0 ? 2 * ncg : ncg) * S;
    // this launch's tiles: the small ones (at most 16 rows) in the MBMAX 1 kernel when the two
    // kernels run on two streams (force_split), or, on one stream, when they fill at least three
    // rounds of three waves per SIMD, so that its last round's tail is short; the rest (or all) in
    // the MBMAX 4 kernel. Up to 16 tokens every tile is small.
    const bool split = p.force_split || p.T <= EVAMX_SMALL_TILE_ROWS || (long)n_small * per_tile >= 3L * (p.gemv_waves * 3 / 4);
    const int n_tiles = MBMAX == 1 ? (split ? n_small : 0) : (split ? n_all - n_small : n_all);
    // the call's items fill the first n_blk workgroups (a multiple of 8, spread over the XCDs)
    const int n_blk = ((n_tiles * per_tile + MF_WAVES - 1) / MF_WAVES + 7) & ~7;
    if ((int)blockIdx.x >= n_blk) return;
    const int blk = xcd_item_block(blockIdx.x, n_blk);
    const int item = __builtin_amdgcn_readfirstlane(blk * MF_WAVES + wave);
    const int ti = item / per_tile;
    if (ti >= n_tiles) return;
    // split: the small tiles from the front of the list, the large ones from the back, each in
    // expert order; otherwise all tiles in chunk order (the tiles of one expert run side by side
    // and share its weight reads in L2)
    const int tile = __builtin_amdgcn_readfirstlane(
        !split ? ti : MBMAX == 1 ? p.tiles[ti] : p.tiles[p.max_chunks - 1 - ti]);
    const int rem = item - ti * per_tile;
    const int ks = rem % S;
    const int pc = rem / S;
    const int proj = which == 0 ? pc / ncg : 2;
    const int cg = pc - (which == 0 ? proj * ncg : 0);
    const int* ch = p.chunks + 8 * tile;
    const int e = __builtin_amdgcn_readfirstlane(ch[0]);
    const int begin = __builtin_amdgcn_readfirstlane(ch[1]);
    const int rows = __builtin_amdgcn_readfirstlane(ch[2]);
    const int k2 = __builtin_amdgcn_readfirstlane(ch[which == 0 ? 3 : 6]);    // gate/up or down rate
    const int* slot_of = p.order + begin;
    const int nslot = moe_nslot(p);
    const int trow = proj == 0 ? EVAMX_TBL_G_TRELLIS : proj == 1 ? EVAMX_TBL_U_TRELLIS : EVAMX_TBL_D_TRELLIS;
    const uint32_t* trellis = (const uint32_t*)(e < 0 ? (const void*)p.sh_ptr[trow]
                                                      : (const void*)p.tables[(size_t)trow * p.tbl_stride + e]);
    GlobalRows src;
    float* part;
    size_t part_stride;
    int nt_n, nch;
    if (which == 0) {
        nch = p.H / 128;
        src = GlobalRows{p.xr + (size_t)proj * p.nslot_max * p.H, (size_t)p.H, p.xsum + (size_t)proj * p.nslot_max * nch, nch};
        part = p.part_gu + ((size_t)ks * 2 + proj) * nslot * p.I;
        part_stride = (size_t)p.I;
        nt_n = p.I / 16;
    } else {
        nch = p.I / 128;
        src = GlobalRows{p.act, (size_t)p.I, p.actsum, nch};
        part = p.part_d + (size_t)ks * nslot * p.H;
        part_stride = (size_t)p.H;
        nt_n = p.H / 16;
    }
    const int kt0 = 8 * (nch * ks / S), kt1 = 8 * (nch * (ks + 1) / S);
    uint32_t* wl = lds[wave];
    switch (k2) {
        case 3: mfma_item_rows<3, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 4: mfma_item_rows<4, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 5: mfma_item_rows<5, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 6: mfma_item_rows<6, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 7: mfma_item_rows<7, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 8: mfma_item_rows<8, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        case 10: mfma_item_rows<10, MBMAX>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, part, part_stride, wl); break;
        default: {
            // unsupported rate (flagged by the grouping): zero partials, so no output reads stale data
            const int lane = threadIdx.x & 63;
            for (int r = 0; r < rows; ++r) {
                float* dst = part + (size_t)slot_of[r] * part_stride + 128 * cg;
                dst[lane] = 0.0f;
                dst[lane + 64] = 0.0f;
            }
        }
    }
}

// The two projection stages as kernels of their own names, so that kernel traces and counter
// runs tell them apart whatever their grids.
template <int MBMAX>
__global__ __launch_bounds__(64 * MF_WAVES) __attribute__((amdgpu_waves_per_eu(MBMAX == 1 ? 3 : 2))) void moe_gate_up_mfma_kernel(MoeParams p)
{
    __shared__ uint32_t lds[MF_WAVES][MF_LDS_WORDS];
    mfma_stage<MBMAX, 0>(p, lds);
}

template <int MBMAX>
__global__ __launch_bounds__(64 * MF_WAVES) __attribute__((amdgpu_waves_per_eu(MBMAX == 1 ? 3 : 2))) void moe_down_mfma_kernel(MoeParams p)
{
    __shared__ uint32_t lds[MF_WAVES][MF_LDS_WORDS];
    mfma_stage<MBMAX, 1>(p, lds);
}

// Side stream of the calling thread on the current device, with its fork and join events, for
// the concurrent MFMA launches of calls of more than 16 tokens. One per thread and device (a
// thread's calls and captures are ordered, so its side stream never joins another thread's
// capture); created on the thread's first such call outside stream capture and kept until the
// process ends, at default priority. nullptr, and the launches stay on the caller's stream, when
// it does not exist and cannot be made (the caller's stream is capturing, a creation failed, an
// earlier error is pending), when it is still joined into a capture other than the caller's, or
// when EVAMX_PREFILL_CONCURRENT=0 is set in the environment (read at each call, to reproduce the
// comparison).
constexpr int SIDE_MAX_DEVICES = 64;

const SideStream* side_stream(hipStream_t stream)
{
    static thread_local SideStream side[SIDE_MAX_DEVICES];
    const char* v = getenv("EVAMX_PREFILL_CONCURRENT");
    if (v && strcmp(v, "0") == 0) return nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SIDE_MAX_DEVICES) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipPeekAtLastError() != hipSuccess) return nullptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    unsigned long long cap_id = 0;
    if (hipStreamGetCaptureInfo(stream, &cap, &cap_id) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    SideStream& ss = side[dev];
    if (ss.s) {
        // a side stream joined into a capture stays in it until the capture ends: fork only
        // from that capture's streams, or, outside any capture, only when it is free
        hipStreamCaptureStatus side_cap = hipStreamCaptureStatusNone;
        unsigned long long side_id = 0;
        if (hipStreamGetCaptureInfo(ss.s, &side_cap, &side_id) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        if (side_cap == hipStreamCaptureStatusActive && (cap != hipStreamCaptureStatusActive || side_id != cap_id))
            return nullptr;
        if (side_cap != hipStreamCaptureStatusNone && side_cap != hipStreamCaptureStatusActive) return nullptr;
        return &ss;
    }
    if (cap != hipStreamCaptureStatusNone) return nullptr;
    SideStream made;
    if (hipStreamCreateWithFlags(&made.s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&made.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&made.join, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        if (made.join) (void)hipEventDestroy(made.join);
        if (made.fork) (void)hipEventDestroy(made.fork);
        if (made.s) (void)hipStreamDestroy(made.s);
        (void)hipGetLastError();
        return nullptr;
    }
    ss = made;
    return &ss;
}

// The largest possible item count of one projection stage: the workspace's tile bound times the
// largest split (an automatic split fills one resident round; gate/up: up to two, see ks_gate_up).
static long mfma_items(const MoeParams& p, int which)
{
    const int ncg = which == 0 ? p.I / 128 : p.H / 128;
    const int kreq = which == 0 ? p.ks_gu : p.ks_d;
    const long per_tile = (long)(which == 0 ? 2 * ncg : ncg);
    const long auto_items = (long)(which == 0 ? 2 : 1) * p.gemv_waves + per_tile;
    return kreq > 0 ? (long)p.max_chunks * per_tile * kreq
                    : (p.max_chunks * per_tile > auto_items ? (long)p.max_chunks * per_tile : auto_items);
}

// Grid of one projection stage in the single-wave form: enough workgroups for mfma_items (a
// multiple of 8); workgroups past the call's items exit at once.
static dim3 mfma_grid(const MoeParams& p, int which)
{
    const long blocks = (mfma_items(p, which) + MF_WAVES - 1) / MF_WAVES;
    return dim3((unsigned)((blocks + 7) & ~7L));
}

int launch_mfma_class(const MoeParams& p, int which, int cls, hipStream_t stream)
{
    MoeParams q = p;
    q.force_split = 1;
    const dim3 grid = mfma_grid(p, which), block(64 * MF_WAVES);
    if (cls == 1)
        launch_timed(which == 0 ? moe_gate_up_mfma_kernel<1> : moe_down_mfma_kernel<1>, grid, block, stream, nullptr, nullptr, q);
    else
        launch_timed(which == 0 ? moe_gate_up_mfma_kernel<4> : moe_down_mfma_kernel<4>, grid, block, stream, nullptr, nullptr, q);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Launch of one projection stage: enough workgroups for the largest possible item count (the
// workspace's tile bound times the largest split); workgroups past the call's items exit at once.
int launch_mfma(const MoeParams& p, int which, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const int ncg = which == 0 ? p.I / 128 : p.H / 128;
    const int kreq = which == 0 ? p.ks_gu : p.ks_d;
    const int kmax = which == 0 ? p.ks_gu_max : p.ks_d_max;
    const long per_tile = (long)(which == 0 ? 2 * ncg : ncg);
    const long items = mfma_items(p, which);
    // tiles of at most 16 rows run in the 16-row kernel (4 waves per SIMD, progress priorities),
    // larger ones in the 64-row kernel; up to 16 tokens every tile is a small one
    // The small-tile launch is skipped when the split can never happen: at most one tile per
    // expert (its remainder) and one shared tile are small, at the largest split count
    const int nslot = p.T * p.topk + (p.has_shared ? p.T : 0);
    const int cap_rows = which == 0 ? p.cap_rows_gu : p.cap_rows_d;
    const int s_max = kreq > 0 ? kreq : (cap_rows / nslot < kmax ? (cap_rows / nslot > 1 ? cap_rows / nslot : 1) : kmax);
    const long max_small = (long)(p.n_local < p.T * p.topk ? p.n_local : p.T * p.topk) + (p.has_shared ? 1 : 0);
    const bool may_split = max_small * per_tile * s_max >= 3L * (p.gemv_waves * 3 / 4);
    auto k16 = which == 0 ? moe_gate_up_mfma_kernel<1> : moe_down_mfma_kernel<1>;
    auto k64 = which == 0 ? moe_gate_up_mfma_kernel<4> : moe_down_mfma_kernel<4>;
    const dim3 grid = mfma_grid(p, which), block(64 * MF_WAVES);
    if (const SideStream* side = p.T > EVAMX_SMALL_TILE_ROWS && p.side_ok ? side_stream(stream) : nullptr) {
        // the tiles of at most 16 rows in the 16-row kernel on the side stream, concurrently with
        // the larger ones in the 64-row kernel on the caller's stream: each fills the other's
        // last round (two kernels of different register budgets cannot share one grid)
        MoeParams q = p;
        q.force_split = 1;
        (void)hipEventRecord(side->fork, stream);
        (void)hipStreamWaitEvent(side->s, side->fork, 0);
        launch_timed(k64, grid, block, stream, start, nullptr, q);
        launch_timed(k16, grid, block, side->s, nullptr, nullptr, q);
        (void)hipEventRecord(side->join, side->s);
        (void)hipStreamWaitEvent(stream, side->join, 0);
        if (stop) (void)hipEventRecord(stop, stream);
    } else if (p.T <= EVAMX_SMALL_TILE_ROWS) {
        launch_timed(k16, grid, block, stream, start, stop, p);
    } else if (!may_split) {
        launch_timed(k64, grid, block, stream, start, stop, p);
    } else {
        launch_timed(k16, grid, block, stream, start, nullptr, p);
        launch_timed(k64, grid, block, stream, nullptr, stop, p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
