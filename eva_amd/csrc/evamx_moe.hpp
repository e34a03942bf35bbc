// Kernel parameter block of the decode MoE pipeline (device pointers into the caller's
// workspace, see moe_workspace_layout in capi.hip).
#pragma once
#include <stdint.h>
#include "../../include/evamx.h"
#include <hip/hip_ext.h>
#include "evamx_device.hpp"

namespace evamx {

constexpr int EVAMX_MAX_EXPERTS = 512;     // pointer-table entries per layer (reference: <= 384)
constexpr int EVAMX_MAX_TOPK = 32;         // reference bound: top_k <= 32 (exl3_moe_coop_kernel.cuh:46)
constexpr int EVAMX_CHUNK = 8;             // slots of one expert per GEMV work item
constexpr int EVAMX_TILE_ROWS = 64;        // slots of one expert per MFMA work item
constexpr int EVAMX_SMALL_TILE_ROWS = 16;  // the same for calls of at most 16 tokens (16-row kernel)
constexpr int EVAMX_MFMA_MIN_ROWS = 3;     // calls with at least this many rows take the MFMA path
                                           // (one decode per tile beats the decode GEMV from 3 rows)

// Pointer-table rows, in the reference's order (ds41/cache.py:1877-1886).
enum {
    EVAMX_TBL_G_TRELLIS = 0, EVAMX_TBL_G_SUH = 1, EVAMX_TBL_G_SVH = 2,
    EVAMX_TBL_U_TRELLIS = 3, EVAMX_TBL_U_SUH = 4, EVAMX_TBL_U_SVH = 5,
    EVAMX_TBL_D_TRELLIS = 6, EVAMX_TBL_D_SUH = 7, EVAMX_TBL_D_SVH = 8,
};

enum { PREP_GROUP = 1, PREP_MOE = 2 };

// Calls of at most this many rows take the decode path (decode GEMVs, work resolved from records).
constexpr int EVAMX_GEMV_MAX_ROWS = EVAMX_MFMA_MIN_ROWS - 1;
// Calls of at most EVAMX_SMALL_ROWS rows and EVAMX_SMALL_SLOTS slots on the MFMA path take the
// one-launch small prepare and the per-token combine.
constexpr int EVAMX_SMALL_SLOTS = 512;
constexpr int EVAMX_SMALL_ROWS = 16;

// Records of the decode path, written by its prepare so that every later kernel resolves its
// work with one load instead of a chain of dependent ones (unit -> chunk -> pointer table ->
// weights). A GEMV wave reads its work unit's record; the activation and combine waves read
// their slot's.
constexpr int EVAMX_NO_UNIT = -2;
struct alignas(128) UnitRec {
    int e;                      // local expert, -1 the shared expert, EVAMX_NO_UNIT past the call's units
    int rows;                   // rows (slots) of the unit's chunk, at most EVAMX_CHUNK
    int k2;                     // 2 x bits of gate and up
    int ubase;                  // first unit of the chunk (a chunk of weight m owns m units)
    int s_gu, s_d;              // k-splits of the chunk's gate/up and down GEMVs
    int k2_d;                   // 2 x bits of down
    int pair;                   // GEMVs of strict calls: 1 this unit's waves take the next unit's
                                // rows too (same expert), -1 the previous unit's take these, 0 alone
    int slot[EVAMX_CHUNK];      // the chunk's slots (entries past rows repeat slot[0])
    uint64_t tr[3];             // gate, up, down trellis
    uint64_t suh[2];            // gate, up input scales
    uint64_t pad1[3];
};
struct alignas(64) SlotRec {
    int active;                 // 0: an inactive slot (zero weight or outside the expert range)
    int shared;                 // 1: a row of the shared expert
    int s_gu, s_d;              // k-splits of the slot's chunk
    float w;                    // routing weight as its fp16 value (1 for the shared expert)
    int pad[3];
    uint64_t g_svh, u_svh, d_suh, d_svh;
};
static_assert(sizeof(UnitRec) == 128 && sizeof(SlotRec) == 64, "record sizes");

struct MoeParams {
    int mode;
    int mfma;                  // 1: expert GEMMs on the MFMA path (chunks of chunk_rows as tiles, each
                               // one work unit of weight 1)
    int chunk_rows;            // rows per GEMV chunk / MFMA tile (0: EVAMX_CHUNK)
    int T, H, I, topk, n_local, n_logits;
    // input rows
    const void* x;
    int x_dtype, x_stride;
    // routing
    const float* logits;
    const float* gate_w;       // router front: logits = x @ gate_w^T into the workspace first (or null)
    const float* sel_bias;
    int score;
    float route_scale;
    int64_t* sel;
    float* weights;            // fp32 weights: output when routing, input otherwise (null: rw16 given)
    half_t* rw16;
    int min_expert, max_expert;
    // experts
    const int64_t* tables;     // [9][tbl_stride]
    int tbl_stride;
    const uint8_t* k2_per_expert;
    int k2_uniform, k2_shared;
    const uint8_t* k2d_per_expert;   // down rates per expert, or null
    int k2d_uniform;                 // uniform down rate when k2d_per_expert is null (0: the gate/up rate)
    int k2_shared_d;                 // the shared expert's down rate
    const half_t* sh_gate_w;         // gated shared expert: fp16 [H], or null
    float* gate_val;                 // [rows]: sigmoid(x_row . sh_gate_w), written by the activation stage
    int has_shared;
    int64_t sh_ptr[9];
    float limit;
    // workspace
    int* err;
    int* local;                // [slots]
    int* order;                // [slots + T]
    int* runs;                 // reference run table [2 + 2*slots_max + 1]
    int slots_max;
    int* chunks;               // [max_chunks][8]: expert (-1 shared), begin, rows, gate/up k2, first
                               // unit, units (cost weight of the chunk, chunk_mult), down k2, 0
    int max_chunks;
    int* unit_chunk;           // [EVAMX_MAX_MULT * max_chunks]: work unit -> chunk
    int* tiles;                // [max_chunks] MFMA tiles by size, each class in expert order: those
                               // of at most 16 rows from the front (meta[3] of them), the rest from
                               // the back
    int* slot_mult;            // [nslot_max]: cost weight of the chunk holding each slot/shared row
    int* meta;                 // [0] n_chunks, [1] n_active, [2] n_units, [3] MFMA tiles of at
                               // most 16 rows
    half_t* xr;                // [2][nslot_max][H] rotated gate/up inputs
    float* xsum;               // [2][nslot_max][H/128] their 128-chunk sums
    half_t* act;               // [nslot_max][I] rotated down inputs
    float* actsum;             // [nslot_max][I/128]
    float* part_gu;            // [ks][2][nslot][I], nslot = rows of this call (moe_nslot)
    float* part_d;             // [ks][nslot][H]
    int nslot_max;
    int ks_gu, ks_d;           // requested k-splits (0: chosen on the device, moe_ks)
    int ks_gu_max, ks_d_max;   // bounds of the automatic choice
    int cap_rows_gu, cap_rows_d;   // partial-buffer capacity in rows (ks * nslot <= cap)
    int gemv_waves;            // grid of the GEMV kernels (waves resident on the device at once)
    int force_split;           // MFMA stages: tiles of at most 16 rows always in the 16-row kernel
    int act_class;             // activation stage: 0 every row; 1 the rows of tiles of at most 16 rows;
                               // 2 the rows of larger tiles (a size class pipelined on its own stream)
    int side_ok;               // host: the MFMA stages may use the thread's side stream (not for the
                               // allocation-free entry point)
    UnitRec* urec;             // decode path: [units_max] work-unit records
    SlotRec* srec;             // decode path: [T * topk + T] slot records (routed slots, shared rows)
    int units_max;             // decode path: work units the launch grids cover (moe_units_max)
    int strict_rows;           // strict batch mode: calls of up to this many rows (0: off) ...
    int strict_ks_gu, strict_ks_d;   // ... run the decode path with these (one-row) k-splits
    int strict;                // this call is strict: every chunk weighs 1 and takes the same splits
    // output
    float* out;                // or null
    int out_stride;
    uint16_t* residual;        // bf16, updated in place, or null
    int residual_stride;
};

// Rates (2 x bits) of local expert e (-1: the shared expert): gate/up, and down (the down tables
// or uniform rate when given, else the gate/up rate).
__device__ __forceinline__ int k2_gu_of(const MoeParams& p, int e)
{
    return e < 0 ? p.k2_shared : p.k2_per_expert ? (int)p.k2_per_expert[e] : p.k2_uniform;
}
__device__ __forceinline__ int k2_d_of(const MoeParams& p, int e)
{
    if (e < 0) return p.k2_shared_d;
    if (p.k2d_per_expert) return (int)p.k2d_per_expert[e];
    return p.k2d_uniform ? p.k2d_uniform : k2_gu_of(p, e);
}

// Rows of the GEMV partial buffers in this call: the routed slots, then the shared expert's rows.
__host__ __device__ __forceinline__ int moe_nslot(const MoeParams& p) { return p.T * p.topk + (p.has_shared ? p.T : 0); }

// Cost weight of a chunk of `rows` rows: its decode is shared by the rows, each row adds its dot
// products, so a chunk of 8 rows costs about three chunks of one. Work is handed out in units
// of weight 1; a chunk of weight m gets m times the k-splits of a one-row chunk.
constexpr int EVAMX_MAX_MULT = 3;
__host__ __device__ __forceinline__ int chunk_mult(int rows) { return rows <= 3 ? 1 : rows <= 6 ? 2 : 3; }
// The weight of a decode-path chunk in this call: 1 in strict mode (every chunk takes the strict
// splits, whatever its rows), else chunk_mult.
__host__ __device__ __forceinline__ int unit_mult(const MoeParams& p, int rows) { return p.strict ? 1 : chunk_mult(rows); }

// Strict calls of more than EVAMX_CHUNK rows pair each expert's chunks (2c, 2c + 1) for the gate/up
// and down launches: one wave decodes the expert's weights once for both chunks' rows (at most 16).
// Their kernels run workgroups of four (or eight) column groups (I / 128 and H / 128 multiples of 4).
__host__ __device__ __forceinline__ bool pair_units(const MoeParams& p)
{
    return p.strict && p.T > EVAMX_CHUNK && (p.I / 128) % 4 == 0 && (p.H / 128) % 4 == 0;
}
// UnitRec::pair of chunk c of nch chunks of one expert.
__host__ __device__ __forceinline__ int unit_pair(int c, int nch) { return (c & 1) ? -1 : (c + 1 < nch ? 1 : 0); }

// Work units of a decode-path call of T rows: at most one per routed slot (a chunk's weight never
// exceeds its rows) and one per EVAMX_CHUNK rows of the shared expert (its chunks weigh 1:
// strict mode, or at most 2 rows).
__host__ __device__ __forceinline__ int moe_units_max(int T, int topk, int has_shared)
{
    return T * topk + (has_shared ? (T + EVAMX_CHUNK - 1) / EVAMX_CHUNK : 0);
}

// K-split choice of a GEMV: `base` splits per work unit, as many as fill the resident grid once
// (or the requested count), a chunk of weight m gets min(base * m, cap) splits (base when the
// split is requested), and cap keeps ks * rows within the partial buffer. Every kernel that
// reads the partials recomputes it from the same inputs.
struct KSplit {
    int base, cap;
};

__host__ __device__ __forceinline__ KSplit moe_ksplit(int req, int items_per_split, int waves, int kmax, int cap_rows, int nslot)
{
    KSplit k;
    k.cap = cap_rows / nslot < kmax ? cap_rows / nslot : kmax;
    if (k.cap < 1) k.cap = 1;
    if (req > 0) {
        k.base = req;
        k.cap = req;
        return k;
    }
    int b = items_per_split > 0 ? waves / items_per_split : 1;
    if (b > k.cap) b = k.cap;
    k.base = b < 1 ? 1 : b;
    return k;
}

__host__ __device__ __forceinline__ int ks_of_chunk(const KSplit& k, int mult)
{
    const int v = k.base * mult;
    return v < k.cap ? v : k.cap;
}

// Waves the automatic split aims for: one resident round (4 per SIMD), except for one-row calls,
// whose GEMV waves aim for two per SIMD. With progress priorities two one-row waves keep a SIMD's
// VALU as busy as four, and half the waves halve the prologues and the partials the next stage
// sums (T=1 82.4 -> 79.6 us); with more rows per chunk two waves per SIMD lose (T=2 116 -> 122,
// T=4 174 -> 255 us).
__host__ __device__ __forceinline__ int split_waves(const MoeParams& p)
{
    return (!p.mfma && p.T == 1) ? p.gemv_waves / 2 : p.gemv_waves;
}

// MFMA gate/up tiles that leave part of one resident round empty unsplit take two splits: with
// items < waves per split, SIMDs hold 3 or 4 equal items, and the ones with 4 set the launch's
// time; two splits even that out (16 tokens at DSv3: gate/up 228-230 -> 224-225 us).
__host__ __device__ __forceinline__ KSplit ks_gate_up(const MoeParams& p, int units)
{
    const int items = units * 2 * (p.I / 128);
    KSplit k = moe_ksplit(p.ks_gu, items, split_waves(p), p.ks_gu_max, p.cap_rows_gu, moe_nslot(p));
    if (p.mfma && p.ks_gu == 0 && k.base == 1 && items < split_waves(p) && k.cap >= 2) k.base = 2;
    return k;
}

__host__ __device__ __forceinline__ KSplit ks_down(const MoeParams& p, int units)
{
    return moe_ksplit(p.ks_d, units * (p.H / 128), split_waves(p), p.ks_d_max, p.cap_rows_d, moe_nslot(p));
}

__host__ __device__ __forceinline__ int chunk_rows_of(const MoeParams& p) { return p.chunk_rows > 0 ? p.chunk_rows : EVAMX_CHUNK; }

int moe_launch(MoeParams& p, hipStream_t stream, void* const* events = nullptr);
// Stage launches of moe_launch, one translation unit each (moe_prepare.hip, moe_gate_up*.hip,
// moe_down.hip, moe_epilogue.hip). start/stop: events that take the first kernel's start and the
// last kernel's end timestamps (nullptr: none).
void launch_router_front(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_prepare(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
// Decode-path gate/up and down (products on the matrix cores): tmax 1 the one-row launches (gate/up
// routes inside), 2 chunks in passes of up to 4 rows, 8 up to 8 rows per pass (gate/up falls back
// to 2-row passes when the column groups are not a multiple of the workgroup's 4 waves).
void launch_gate_up_decode(const MoeParams& p, int tmax, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_gate_up_decode8(const MoeParams& p, long waves, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_gate_up_decode16(const MoeParams& p, long waves, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_gate_up_decode4(const MoeParams& p, bool group, dim3 grid, hipStream_t stream, hipEvent_t start,
                            hipEvent_t stop);
void launch_down_decode(const MoeParams& p, int tmax, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_down_decode16(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_act(const MoeParams& p, int nslot, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
void launch_act_class(const MoeParams& p, int cls, hipStream_t stream);
void launch_combine(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
// Kernel launch that, given events, records the kernel's own start and end timestamps in them
// (hipExtLaunchKernel), as a profiler's kernel trace reports them; plain launch otherwise.
template <typename... KArgs, typename... Args>
inline void launch_timed(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, hipEvent_t start,
                         hipEvent_t stop, Args... args)
{
    if (start || stop)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
}

int launch_mfma(const MoeParams& p, int which, hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// One size class of an MFMA stage on its own: cls 1 the tiles of at most 16 rows (16-row kernel),
// cls 2 the larger ones (64-row kernel); both read the split tile list.
int launch_mfma_class(const MoeParams& p, int which, int cls, hipStream_t stream);
// The calling thread's side stream on the current device with its fork and join events, or
// nullptr (see moe_prefill.hip).
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
const SideStream* side_stream(hipStream_t stream);
int moe_prepare_only(MoeParams& p, hipStream_t stream);
int launch_router_logits(const MoeParams& p, float* logits, hipStream_t stream);
bool moe_small_path(int T, int topk);

}  // namespace evamx
