/*
 * evamx: MI355X (gfx950) implementation of eva's cooperative EXL3 MoE expert path, as a
 * C ABI. Plain pointers and sizes; every pointer argument documented "device" is a HIP device
 * pointer; `stream` is a hipStream_t. No entry point allocates or synchronises with the host,
 * so a forward call can be captured into a hipGraph. Errors are returned as negative codes
 * with a message from evamx_last_error() (thread-local).
 *
 * Reference interfaces replaced (paths under runtime/ds41/ of the eva repository):
 *   evamx_exl3_dequant       decoded fp16 weights of an EXL3 projection:
 *                            csrc/moe_coop3072/vendor/quant/exl3_dq.cuh:96-330 with
 *                            codebook.cuh:86-99 (the "decoded fp16 weight" contract)
 *   evamx_exl3_linear        ELinear.forward -> LinearEXL3 (exl3_linear.py:97-131,134-154),
 *                            kernel csrc/moe_coop3072/vendor/quant/exl3_gemv_kernel.cuh:195-491
 *   evamx_router_logits      the gate GEMV of Block.route, stable_linear(x.float(), gate_w)
 *                            (model.py:158-165,404-409; stable_linear_runtime "router" dispatch)
 *   evamx_route_topk         Block.route (model.py:404-416) with the stable tie rule of
 *                            _stable_topk_indices (model.py:940-953)
 *   evamx_prepare_routes     CoopRunner3072.prepare_routes -> pybind prepare_routes
 *                            (moe_coop3072.py:321-358; csrc/moe_coop3072/moe_coop3072.cu:149-174)
 *   evamx_moe_forward        CoopRunner*.run -> pybind run / exllamav3_ext.exl3_moe_coop
 *                            (moe_coop.py:42-69; moe_coop3072.py:261-319;
 *                            csrc/moe_coop3072/moe_coop3072.cu:73-145;
 *                            csrc/moe_coop3072/vendor/quant/exl3_moe_coop.cuh:115-152),
 *                            plus the shared expert added by Block.experts (model.py:418-452,498)
 *   evamx_moe_workspace_bytes  WorkspaceLayout.scratch_bytes / exl3_moe_coop_ctr_len
 *                            (moe_coop3072.py:120-152; exl3_moe_coop.cuh:154-159)
 */
#ifndef EVAMX_H
#define EVAMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* evamx_stream_t; /* hipStream_t */

enum { EVAMX_OK = 0, EVAMX_EINVAL = -1, EVAMX_ELAUNCH = -2, EVAMX_ENOSPACE = -3 };
enum { EVAMX_DTYPE_F16 = 0, EVAMX_DTYPE_BF16 = 1 };
enum { EVAMX_SCORE_SIGMOID = 0, EVAMX_SCORE_SQRT_SOFTPLUS = 1 };
/* Device-side error flags (sticky bits in the workspace, read with evamx_moe_flags_ptr). */
enum { EVAMX_ERR_EXPERT_RANGE = 1, EVAMX_ERR_RATE = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* evamx_last_error(void);
/* ABI version of this library (incremented on incompatible changes). */
int evamx_abi_version(void);

/* ---- EXL3 decode ------------------------------------------------------------------------ */

/* Decode one EXL3 projection to fp16 W[in][out] (row-major), bit-exact with the reference
 * MUL1 codebook. trellis: device int16 [in/16][out/16][16*bits] (16b+8 at rate b+0.5).
 * bits in {1..8} or {1.5, 2.5, 3.5}. */
int evamx_exl3_dequant(const void* trellis, int in_features, int out_features, float bits,
                       void* w_fp16, evamx_stream_t stream);

/* ---- single EXL3 linear (fp16 in, fp16 out) ---------------------------------------------- */

size_t evamx_exl3_linear_workspace_bytes(int rows, int in_features, int out_features);

/* y[rows][out] = svh * H(W^T H(x * suh)) with the reference's fp16 rounding points.
 * rows in 1..65536 (up to 16 rows a decode GEMV, beyond it MFMA tiles; within each a row's result
 * does not depend on how many rows share the call); in/out multiples of 128; bits in
 * {1.5,2,2.5,3,3.5,4,5}. All pointers device. Up to 2 rows the call is one launch: the
 * workgroups of each 128-column group meet at an arrival counter kept in the workspace, which may
 * hold anything before its first use (the call then counts with compare-and-swap) and is left at
 * rest by every call, graph replays included. Calls that share a workspace must not overlap. */
int evamx_exl3_linear(const void* x_fp16, int rows, int in_features, int out_features,
                      const void* trellis, const void* suh_fp16, const void* svh_fp16, float bits,
                      void* y_fp16, void* workspace, size_t workspace_bytes, evamx_stream_t stream);

/* ---- router ------------------------------------------------------------------------------ */

/* logits[r][e] = sum_k float(x[r][k]) * gate_w[e][k] (fp32): the router gate GEMV of
 * Block.route, stable_linear(x.float(), gate_w) (model.py:158-165,404-409). Each row's sums run
 * in one fixed order whatever `rows` is (batch invariant). x: device fp16/bf16 [rows][x_stride];
 * gate_w: device fp32 [n_experts][hidden], 16-byte aligned; hidden a multiple of 4. */
int evamx_router_logits(const void* x, int x_dtype, int x_stride, int rows, const float* gate_w,
                        int n_experts, int hidden, float* logits, evamx_stream_t stream);

/* indices[r][j], weights[r][j] (fp32) and rw_fp16[r][j] = fp16(weights) for the top `topk`
 * experts of each row of logits [rows][n_experts]: selection key score(z) + sel_bias (or z
 * itself for sigmoid without a bias), ties to the lower index, slots ordered by descending
 * key; weights = score / (sum + 1e-20) * route_scale. sel_bias: device [n_experts] or NULL. */
int evamx_route_topk(const float* logits, const float* sel_bias, int rows, int n_experts, int topk,
                     int score_fn, float route_scale, int64_t* indices, float* weights, void* rw_fp16,
                     evamx_stream_t stream);

/* ---- slot grouping (the reference's run table) ------------------------------------------- */

size_t evamx_prepare_routes_workspace_bytes(int capacity, int topk);

/* runs: device int32 [2 + 2*capacity*topk + 1] =
 *   [n_runs, 0, run_start[0..capacity*topk], order[capacity*topk]] with unused entries zero:
 * active slots (fp16 weight != 0) sorted by (expert, slot), cut at an expert change or every
 * 8 slots. Expert indices outside [0, n_local) set EVAMX_ERR_EXPERT_RANGE in the workspace's
 * flag word (evamx_prepare_routes_flags_ptr) and make the slot inactive. */
int evamx_prepare_routes(const int64_t* sel, const void* rw_fp16, int rows, int topk, int capacity,
                         int n_local, int32_t* runs, void* workspace, size_t workspace_bytes,
                         evamx_stream_t stream);
int32_t* evamx_prepare_routes_flags_ptr(void* workspace);

/* ---- MoE layer forward --------------------------------------------------------------------- */

typedef struct evamx_moe_shape {
    int32_t rows_max;     /* token rows per call (capacity) */
    int32_t hidden;       /* H, multiple of 128 */
    int32_t inter;        /* I, multiple of 128 */
    int32_t topk;         /* <= 32 */
    int32_t n_local;      /* pointer-table entries, <= 512 */
    int32_t has_shared;   /* 1: a shared expert is added to every row */
    int32_t ksplit_gu;    /* k-splits of the gate/up GEMV (0: chosen per call on the device
                             from the number of expert chunks, to fill the GPU once) */
    int32_t ksplit_down;  /* k-splits of the down GEMV (0: likewise) */
    /* ABI 5. Strict batch mode, the reference's DS41_STRICT_BATCH (moe_coop.py:17-22, which pins
     * EXL3_MOE_COOP_WIDE=0 / EXL3_MOE_COOP_KSPLIT=1 so that "target and verification arithmetic"
     * stay identical; cache.py:2088-2091), bounded by its verification row limit
     * (verification.py:15-30). 0: every call picks its product path and k-splits from its row
     * count (fastest). 1..EVAMX_STRICT_MAX_ROWS (with strict_rows * topk <= EVAMX_STRICT_MAX_SLOTS):
     * calls of 1..strict_rows rows run every row through the arithmetic of a one-row call (the
     * decode GEMV with the k-splits a one-row call picks, or ksplit_gu/ksplit_down when given), so
     * each row's output is bit-identical whatever the call's row count in that range. Calls of
     * more rows keep the automatic geometry. */
    int32_t strict_rows;
} evamx_moe_shape;

enum { EVAMX_STRICT_MAX_ROWS = 64, EVAMX_STRICT_MAX_SLOTS = 256 };

typedef struct evamx_moe_args {
    evamx_moe_shape shape;
    int32_t rows;                 /* T, 1..rows_max */
    const void* x;                /* device [rows][x_stride] fp16 or bf16, 4-byte aligned */
    int32_t x_dtype;              /* EVAMX_DTYPE_* */
    int32_t x_stride;             /* elements; even, >= hidden */
    /* routing: logits != NULL routes on device and writes sel/weights/rw_fp16; otherwise
     * sel and weights (fp32) are inputs, or sel and rw_fp16 when weights == NULL */
    const float* logits;          /* device [rows][n_logits] or NULL */
    const float* sel_bias;        /* device [n_logits] or NULL */
    int32_t n_logits;             /* experts in the logits (= n_local without expert ranges) */
    int32_t score_fn;             /* EVAMX_SCORE_* */
    float route_scale;
    int64_t* sel;                 /* device [rows][topk] */
    float* weights;               /* device [rows][topk] fp32, or NULL */
    void* rw_fp16;                /* device [rows][topk] fp16, or NULL (workspace copy) */
    int32_t min_expert;           /* -1: no expert range; else sel in [min, max) is local */
    int32_t max_expert;
    /* experts */
    const int64_t* tables;        /* device int64 [9][n_local]: g_trellis, g_suh, g_svh,
                                     u_trellis, u_suh, u_svh, d_trellis, d_suh, d_svh */
    const uint8_t* k2_per_expert; /* device [n_local], 2*bits per expert (3..8 or 10), or NULL;
                                     another value sets EVAMX_ERR_RATE and the expert adds 0 */
    float bits;                   /* uniform rate when k2_per_expert is NULL: 1.5 .. 4 in steps
                                     of 0.5, or 5 */
    const int64_t* shared;        /* HOST array of 9 device pointers (table order) or NULL */
    float shared_bits;
    float limit;                  /* SwiGLU limit (0: none) */
    /* output: out[r][0..hidden) = routed (slot order, fp32) + shared */
    float* out;                   /* device, or NULL when residual is given */
    int32_t out_stride;           /* elements; >= hidden */
    void* workspace;              /* device, evamx_moe_workspace_bytes(&shape) bytes */
    size_t workspace_bytes;
    /* optional: 10 hipEvent_t for the 5 stages (prepare, gate/up, activation, down,
     * combine): events[2k] takes the start timestamp of stage k's first kernel and
     * events[2k+1] the end timestamp of its last (kernel timestamps, hipExtLaunchKernel);
     * NULL for none. A 1-row call routes inside its gate/up launch: its prepare stage is the
     * router front alone when gate_w is given, and otherwise has no kernel and records no
     * events. */
    void* const* events;
    /* optional residual stream: bf16 [rows][residual_stride], updated in place to
     * bf16(residual + bf16(out)) (the layer output cast to the activation dtype and added,
     * model.py:499); may be the x of this call. NULL for none. */
    void* residual;
    int32_t residual_stride;      /* elements; >= hidden */
    /* optional router front (Block.route's x.float() @ gate_w.T, model.py:404-409 with the
     * per-row stable_linear of model.py:158-165): device fp32 [n_logits][hidden]; when set and
     * logits == NULL, each row's logits are computed on the device in fp32 with a fixed
     * reduction order (independent of the batch) and routed as above. NULL for none. */
    const float* gate_w;
    /* ABI 4. Optional rate of the down projections when it differs from gate/up (the reference
     * launcher takes K_gu for gate and up and K_d for down, vendor/quant/exl3_moe_coop.cuh:80-83):
     * a uniform bits_down, or per expert k2_down_per_expert (device [n_local], 2*bits); 0 / NULL:
     * the gate/up rate. shared_bits_down likewise for the shared expert (0: shared_bits). */
    float bits_down;
    const uint8_t* k2_down_per_expert;
    float shared_bits_down;
    /* ABI 4. Optional gated shared expert (exl3_moe_coop_kernel.cuh:881-903,942-948): device fp16
     * [hidden], 4-byte aligned; each row's shared term is scaled by sigmoid(x_row . shared_gate_w)
     * (fp32 dot of the fp16 row) before it is added. NULL: ungated. */
    const void* shared_gate_w;
} evamx_moe_args;

size_t evamx_moe_workspace_bytes(const evamx_moe_shape* shape);
/* No counterpart in the reference (its runners own their scratch tensors). For callers that
 * cannot allocate device memory (code under hipGraph capture, serving loops that forbid
 * hipMalloc): evamx_moe_forward with args->workspace == NULL and workspace_bytes == 0, run on
 * the library's fixed device scratch of 64 MiB per GPU (held until the process ends). Shapes
 * whose evamx_moe_workspace_bytes exceeds 64 MiB are rejected with EVAMX_ENOSPACE (DSv3 decode
 * needs 44-53 MiB for 1-32 rows). Calls no allocator. All calls on one GPU share its scratch:
 * calls that overlap on one GPU race. Device-side error flags are not reported by this entry
 * point (flagged slots are skipped, as in evamx_moe_forward). */
int evamx_moe_forward_static(const evamx_moe_args* args, evamx_stream_t stream);
/* Zero the workspace's sticky flag word (a kernel, not a memset: capture-safe). Call once
 * after allocating the workspace. */
int evamx_moe_workspace_init(const evamx_moe_shape* shape, void* workspace, evamx_stream_t stream);
int evamx_moe_forward(const evamx_moe_args* args, evamx_stream_t stream);
/* Device pointers into a workspace: the run table of the last forward (layout of
 * evamx_prepare_routes with capacity = rows_max) and the sticky flag word. */
int32_t* evamx_moe_runs_ptr(const evamx_moe_shape* shape, void* workspace);
int32_t* evamx_moe_flags_ptr(const evamx_moe_shape* shape, void* workspace);
/* The fp32 router logits [rows][n_logits] the last forward computed from gate_w (the router
 * stable_linear of model.py:404-409 / stable_linear_runtime's "router" dispatch); undefined after
 * a forward given logits. */
float* evamx_moe_logits_ptr(const evamx_moe_shape* shape, void* workspace);
/* The rotated gate/up inputs fp16(H128(fp16(x) * suh)) the last forward of 3 or more rows wrote,
 * the activations the reference's rotation kernel (exl3_moe_coop_kernel.cuh:613-671) hands to its
 * gate and up GEMVs: fp16 [2][nslot_max][hidden], projection 0 gate and 1 up, routed slot
 * row * topk + k for each active slot, shared-expert row r at rows * topk + r, with nslot_max =
 * rows_max * topk (+ rows_max with a shared expert). Undefined for inactive slots and after calls
 * of 1-2 rows, whose waves rotate their inputs in LDS. */
const void* evamx_moe_rotated_ptr(const evamx_moe_shape* shape, void* workspace);

/* ---- measurement --------------------------------------------------------------------------- */

/* No counterpart in the reference: a benchmark kernel for the arithmetic bound of the decode
 * GEMV. `waves` waves each decode `iters` k-slices (32 weights per lane) of register-resident
 * trellis words at rate `bits` with the GEMV's matrix-core products (eight 4x4x4 MFMA blocks per
 * slice and row group), the GEMV's per-weight instruction mix without its memory traffic; time
 * it with events on `stream`.
 * Weights decoded = waves * 64 * 32 * iters. sink: device float[256] (written only to keep the
 * work observable). */
int evamx_bench_decode(float bits, int waves, int iters, float* sink, evamx_stream_t stream);

/* No counterpart in the reference: a benchmark kernel for the memory-side bound of a decode
 * GEMV launch. `waves` waves (a multiple of ncg) each read `rows` chunks of 1 KiB (64 lanes x 16
 * bytes, non-temporal, four in flight): wave w reads byte (w % ncg) * 1024 of rows
 * (w / ncg) * rows .. + rows - 1 of buf, whose rows are ncg KiB long. With ncg = columns / 128,
 * rows = the k-slices of one split and waves = the launch's waves this is the bytes of that
 * launch at 4 bits in its access shape, without the decode. Reads waves * rows KiB, which must
 * fit in `bytes`; time it with events on `stream`. sink: device float[64] (written only to keep
 * the loads observable). */
int evamx_bench_read(const void* buf, size_t bytes, int ncg, int rows, int waves, float* sink, evamx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EVAMX_H */
