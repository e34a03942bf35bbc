// C ABI of libevamx: argument validation, workspace layouts and launches (include/evamx.h).
//
// Validation mirrors the reference's synchronous checks (csrc/moe_coop3072/moe_coop3072.cu:76-124,
// moe_coop3072.py:261-297) except the host-synchronising expert bounds check, which becomes a
// device-side flag (the slot is then treated as inactive, so no pointer outside the table is
// ever read).
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "evamx_internal.hpp"
#include "evamx_moe.hpp"

namespace evamx {

static thread_local char g_err[512];

void set_error(const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

static int rate_k2(float bits)
{
    if (!std::isfinite(bits)) return -1;
    const float k2 = bits * 2.0f;
    const int i = (int)lrintf(k2);
    if (std::fabs(k2 - (float)i) > 1e-4f) return -1;
    if (i >= 2 && i <= 16 && !(i & 1)) return i;           // 1..8
    if (i == 3 || i == 5 || i == 7) return i;               // 1.5, 2.5, 3.5
    return -1;
}

static bool gemv_rate(int k2) { return gemv_k2_supported(k2); }   // 1.5 .. 4, 5 bits

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

struct MoeLayout {
    size_t flags, meta, local, order, runs, chunks, unit_chunk, tiles, slot_mult, rw16, urec, srec, gate_val, logits, xr,
        xsum, act, actsum, part_gu, part_d, total;
    int slots_max, nslot_max, max_chunks, ks_gu, ks_d, ks_gu_max, ks_d_max, cap_rows_gu, cap_rows_d;
    int strict_ks_gu, strict_ks_d;
};

// Rows of GEMV partials a workspace holds when the k-split is chosen on the device: enough
// for the splits that fill the grid at small batches (ks * rows <= this), and one split of
// every row of a full batch.
constexpr int EVAMX_AUTO_PART_ROWS = 1024;

// Waves the GEMV kernels keep resident: 4 per SIMD (their register budget) on every CU.
static int gemv_waves()
{
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus * 4 * 4;
    }
    return cached[dev];
}

static bool shape_ok(const evamx_moe_shape* s)
{
    if (!s) { set_error("evamx: null shape"); return false; }
    if (s->rows_max < 1 || s->rows_max > 65536) { set_error("evamx: rows_max %d outside 1..65536", s->rows_max); return false; }
    if (s->hidden < 128 || s->hidden % 128 || s->inter < 128 || s->inter % 128) {
        set_error("evamx: hidden %d and inter %d must be positive multiples of 128", s->hidden, s->inter);
        return false;
    }
    if (s->topk < 1 || s->topk > EVAMX_MAX_TOPK) { set_error("evamx: topk %d outside 1..%d", s->topk, EVAMX_MAX_TOPK); return false; }
    if (s->n_local < 1 || s->n_local > EVAMX_MAX_EXPERTS) {
        set_error("evamx: n_local %d outside 1..%d", s->n_local, EVAMX_MAX_EXPERTS);
        return false;
    }
    if (s->ksplit_gu < 0 || s->ksplit_gu > 64 || s->ksplit_down < 0 || s->ksplit_down > 64) {
        set_error("evamx: ksplit outside 0..64");
        return false;
    }
    if ((long)s->rows_max * s->topk > 65536) { set_error("evamx: rows_max*topk above 65536"); return false; }
    if (s->strict_rows < 0 || s->strict_rows > EVAMX_STRICT_MAX_ROWS || s->strict_rows * s->topk > EVAMX_STRICT_MAX_SLOTS) {
        set_error("evamx: strict_rows %d outside 0..%d (at most %d slots)", s->strict_rows, EVAMX_STRICT_MAX_ROWS,
                  EVAMX_STRICT_MAX_SLOTS);
        return false;
    }
    return true;
}

// Rows of a call that the decode path serves with this shape: up to EVAMX_GEMV_MAX_ROWS, and up
// to strict_rows in strict mode.
static int decode_rows(const evamx_moe_shape* s)
{
    const int r = s->strict_rows > EVAMX_GEMV_MAX_ROWS ? s->strict_rows : EVAMX_GEMV_MAX_ROWS;
    return s->rows_max < r ? s->rows_max : r;
}

// K-splits of strict mode: the ones a one-row call picks on its own (split_waves / moe_ksplit at
// T = 1 on the decode path: the one-row unit count, half a resident round of waves), or the
// requested ones; both depend on the shape and the device only, never on the call's rows.
static void strict_splits(const evamx_moe_shape* s, int kgu_max, int kd_max, int& gu, int& d)
{
    const int units1 = s->topk + (s->has_shared ? 1 : 0);
    const int waves = gemv_waves() / 2;
    auto pick = [&](int req, int items, int kmax) {
        if (req > 0) return req < kmax ? req : kmax;
        int b = waves / items;
        if (b > kmax) b = kmax;
        return b < 1 ? 1 : b;
    };
    gu = pick(s->ksplit_gu, units1 * 2 * (s->inter / 128), kgu_max);
    d = pick(s->ksplit_down, units1 * (s->hidden / 128), kd_max);
}

static MoeLayout moe_layout(const evamx_moe_shape* s)
{
    MoeLayout L;
    L.slots_max = s->rows_max * s->topk;
    L.nslot_max = L.slots_max + (s->has_shared ? s->rows_max : 0);
    const int routed_chunks = (L.slots_max < s->n_local ? L.slots_max : s->n_local) + L.slots_max / EVAMX_CHUNK;
    L.max_chunks = routed_chunks + (s->has_shared ? (s->rows_max + EVAMX_CHUNK - 1) / EVAMX_CHUNK : 0);
    L.ks_gu_max = s->hidden / 128 < 32 ? s->hidden / 128 : 32;
    L.ks_d_max = s->inter / 128 < 32 ? s->inter / 128 : 32;
    L.ks_gu = s->ksplit_gu > L.ks_gu_max ? L.ks_gu_max : s->ksplit_gu;
    L.ks_d = s->ksplit_down > L.ks_d_max ? L.ks_d_max : s->ksplit_down;
    const int auto_rows = L.nslot_max > EVAMX_AUTO_PART_ROWS ? L.nslot_max : EVAMX_AUTO_PART_ROWS;
    L.cap_rows_gu = L.ks_gu ? L.ks_gu * L.nslot_max : auto_rows;
    L.cap_rows_d = L.ks_d ? L.ks_d * L.nslot_max : auto_rows;
    const int dr = decode_rows(s);
    L.strict_ks_gu = L.strict_ks_d = 0;
    if (s->strict_rows > 0) {
        // strict calls keep the one-row splits at every row count up to strict_rows
        strict_splits(s, L.ks_gu_max, L.ks_d_max, L.strict_ks_gu, L.strict_ks_d);
        const int sr = s->rows_max < s->strict_rows ? s->rows_max : s->strict_rows;
        const int nslot_s = sr * s->topk + (s->has_shared ? sr : 0);
        if (L.cap_rows_gu < L.strict_ks_gu * nslot_s) L.cap_rows_gu = L.strict_ks_gu * nslot_s;
        if (L.cap_rows_d < L.strict_ks_d * nslot_s) L.cap_rows_d = L.strict_ks_d * nslot_s;
    }
    size_t o = 0;
    L.flags = o;   o = al256(o + 64 * 4);     // first: evamx_moe_forward_static zeroes offset 0 of its scratch
    L.meta = o;    o = al256(o + 64 * 4);
    L.local = o;   o = al256(o + (size_t)L.slots_max * 4);
    L.order = o;   o = al256(o + (size_t)L.nslot_max * 4);
    L.runs = o;    o = al256(o + (size_t)(2 + 2 * L.slots_max + 1) * 4);
    L.chunks = o;  o = al256(o + (size_t)L.max_chunks * 32);
    L.unit_chunk = o; o = al256(o + (size_t)EVAMX_MAX_MULT * L.max_chunks * 4);
    L.tiles = o;   o = al256(o + (size_t)L.max_chunks * 4);
    L.slot_mult = o; o = al256(o + (size_t)L.nslot_max * 4);
    L.rw16 = o;    o = al256(o + (size_t)L.slots_max * 2);
    // decode-path records of calls of at most dr rows: a unit per routed slot at most (a chunk's
    // weight never exceeds its rows) and the shared expert's chunks of EVAMX_CHUNK rows
    L.urec = o; o = al256(o + (size_t)moe_units_max(dr, s->topk, s->has_shared) * sizeof(UnitRec));
    L.srec = o; o = al256(o + (size_t)dr * (s->topk + 1) * sizeof(SlotRec));
    L.gate_val = o; o = al256(o + (size_t)s->rows_max * 4);
    L.logits = o;  o = al256(o + (size_t)s->rows_max * EVAMX_MAX_EXPERTS * 4);
    L.xr = o;      o = al256(o + (size_t)2 * L.nslot_max * s->hidden * 2);
    L.xsum = o;    o = al256(o + (size_t)2 * L.nslot_max * (s->hidden / 128) * 4);
    L.act = o;     o = al256(o + (size_t)L.nslot_max * s->inter * 2);
    L.actsum = o;  o = al256(o + (size_t)L.nslot_max * (s->inter / 128) * 4);
    L.part_gu = o; o = al256(o + (size_t)L.cap_rows_gu * 2 * s->inter * 4);
    L.part_d = o;  o = al256(o + (size_t)L.cap_rows_d * s->hidden * 4);
    L.total = o;
    return L;
}

__global__ void fill_i32_kernel(int* p, int n, int v)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

void launch_fill_i32(int* p, int n, int v, hipStream_t stream)
{
    hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, p, n, v);
}

int launched(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("evamx: %s launch failed: %s", what, hipGetErrorString(e));
        return EVAMX_ELAUNCH;
    }
    return EVAMX_OK;
}

}  // namespace evamx

using namespace evamx;

#define EVAMX_REQUIRE(cond, ...)              \
    do {                                      \
        if (!(cond)) {                        \
            set_error(__VA_ARGS__);           \
            return EVAMX_EINVAL;              \
        }                                     \
    } while (0)

extern "C" const char* evamx_last_error(void) { return g_err; }

extern "C" int evamx_abi_version(void) { return 5; }

extern "C" int evamx_exl3_dequant(const void* trellis, int in_features, int out_features, float bits, void* w_fp16,
                                  evamx_stream_t stream)
{
    g_err[0] = 0;
    const int k2 = rate_k2(bits);
    EVAMX_REQUIRE(trellis && w_fp16, "evamx_exl3_dequant: null pointer");
    EVAMX_REQUIRE(k2 > 0, "evamx_exl3_dequant: unsupported bit rate %g", (double)bits);
    EVAMX_REQUIRE(in_features >= 16 && out_features >= 16 && in_features % 16 == 0 && out_features % 16 == 0,
                  "evamx_exl3_dequant: in/out (%d, %d) must be positive multiples of 16", in_features, out_features);
    launch_dequant(trellis, in_features, out_features, k2, w_fp16, false, (hipStream_t)stream);
    return launched("dequant");
}

extern "C" size_t evamx_exl3_linear_workspace_bytes(int rows, int in_features, int out_features)
{
    if (rows < 1 || rows > 65536 || in_features < 128 || out_features < 128) return 0;
    return linear_workspace(rows, in_features, out_features, nullptr, nullptr);
}

extern "C" int evamx_exl3_linear(const void* x_fp16, int rows, int in_features, int out_features, const void* trellis,
                                 const void* suh_fp16, const void* svh_fp16, float bits, void* y_fp16, void* workspace,
                                 size_t workspace_bytes, evamx_stream_t stream)
{
    g_err[0] = 0;
    const int k2 = rate_k2(bits);
    EVAMX_REQUIRE(x_fp16 && trellis && suh_fp16 && svh_fp16 && y_fp16 && workspace, "evamx_exl3_linear: null pointer");
    EVAMX_REQUIRE(rows >= 1 && rows <= 65536, "evamx_exl3_linear: rows %d outside 1..65536", rows);
    EVAMX_REQUIRE(in_features >= 128 && out_features >= 128 && in_features % 128 == 0 && out_features % 128 == 0,
                  "evamx_exl3_linear: in/out (%d, %d) must be positive multiples of 128", in_features, out_features);
    EVAMX_REQUIRE(gemv_rate(k2), "evamx_exl3_linear: bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", (double)bits);
    const size_t need = linear_workspace(rows, in_features, out_features, nullptr, nullptr);
    EVAMX_REQUIRE(rows > 16 || need < ((size_t)1 << 31),
                  "evamx_exl3_linear: %d x %d with %d rows exceeds the decode path's 2 GiB of partials", in_features,
                  out_features, rows);
    if (workspace_bytes < need) {
        set_error("evamx_exl3_linear: workspace %zu bytes < %zu", workspace_bytes, need);
        return EVAMX_ENOSPACE;
    }
    launch_linear(x_fp16, rows, in_features, out_features, trellis, suh_fp16, svh_fp16, k2, y_fp16, workspace,
                  (hipStream_t)stream);
    return launched("linear");
}

extern "C" int evamx_route_topk(const float* logits, const float* sel_bias, int rows, int n_experts, int topk,
                                int score_fn, float route_scale, int64_t* indices, float* weights, void* rw_fp16,
                                evamx_stream_t stream)
{
    g_err[0] = 0;
    EVAMX_REQUIRE(logits && indices && weights && rw_fp16, "evamx_route_topk: null pointer");
    EVAMX_REQUIRE(rows >= 1 && rows <= 65536, "evamx_route_topk: rows %d outside 1..65536", rows);
    EVAMX_REQUIRE(n_experts >= 1 && n_experts <= EVAMX_MAX_EXPERTS, "evamx_route_topk: n_experts %d outside 1..%d",
                  n_experts, EVAMX_MAX_EXPERTS);
    EVAMX_REQUIRE(topk >= 1 && topk <= EVAMX_MAX_TOPK && topk <= n_experts, "evamx_route_topk: topk %d invalid", topk);
    EVAMX_REQUIRE(score_fn == EVAMX_SCORE_SIGMOID || score_fn == EVAMX_SCORE_SQRT_SOFTPLUS,
                  "evamx_route_topk: unknown score function %d", score_fn);
    EVAMX_REQUIRE(std::isfinite(route_scale), "evamx_route_topk: route_scale must be finite");
    MoeParams p;
    memset(&p, 0, sizeof p);
    p.mode = 0;
    p.T = rows; p.topk = topk; p.n_logits = n_experts;
    p.logits = logits; p.sel_bias = sel_bias; p.score = score_fn; p.route_scale = route_scale;
    p.sel = indices; p.weights = weights; p.rw16 = (half_t*)rw_fp16;
    moe_prepare_only(p, (hipStream_t)stream);
    return launched("route_topk");
}

extern "C" int evamx_router_logits(const void* x, int x_dtype, int x_stride, int rows, const float* gate_w,
                                   int n_experts, int hidden, float* logits, evamx_stream_t stream)
{
    g_err[0] = 0;
    EVAMX_REQUIRE(x && gate_w && logits, "evamx_router_logits: null pointer");
    EVAMX_REQUIRE(x_dtype == EVAMX_DTYPE_F16 || x_dtype == EVAMX_DTYPE_BF16, "evamx_router_logits: x_dtype %d", x_dtype);
    EVAMX_REQUIRE(rows >= 1 && rows <= 65536, "evamx_router_logits: rows %d outside 1..65536", rows);
    EVAMX_REQUIRE(n_experts >= 1 && n_experts <= EVAMX_MAX_EXPERTS, "evamx_router_logits: n_experts %d outside 1..%d",
                  n_experts, EVAMX_MAX_EXPERTS);
    EVAMX_REQUIRE(hidden >= 4 && hidden % 4 == 0 && x_stride >= hidden,
                  "evamx_router_logits: hidden %d must be a positive multiple of 4 and x_stride >= hidden", hidden);
    EVAMX_REQUIRE(((uintptr_t)gate_w & 15) == 0, "evamx_router_logits: gate_w must be 16-byte aligned");
    MoeParams p;
    memset(&p, 0, sizeof p);
    p.T = rows; p.H = hidden; p.n_logits = n_experts;
    p.x = x; p.x_dtype = x_dtype; p.x_stride = x_stride;
    p.gate_w = gate_w;
    launch_router_logits(p, logits, (hipStream_t)stream);
    return launched("router_logits");
}

extern "C" size_t evamx_prepare_routes_workspace_bytes(int capacity, int topk)
{
    if (capacity < 1 || topk < 1) return 0;
    return 256 + al256((size_t)capacity * topk * 4);
}

extern "C" int32_t* evamx_prepare_routes_flags_ptr(void* workspace) { return (int32_t*)workspace; }

extern "C" int evamx_prepare_routes(const int64_t* sel, const void* rw_fp16, int rows, int topk, int capacity,
                                    int n_local, int32_t* runs, void* workspace, size_t workspace_bytes,
                                    evamx_stream_t stream)
{
    g_err[0] = 0;
    EVAMX_REQUIRE(sel && rw_fp16 && runs && workspace, "evamx_prepare_routes: null pointer");
    EVAMX_REQUIRE(topk >= 1 && topk <= EVAMX_MAX_TOPK, "evamx_prepare_routes: topk %d outside 1..%d", topk, EVAMX_MAX_TOPK);
    EVAMX_REQUIRE(capacity >= 1 && (long)capacity * topk <= 65536, "evamx_prepare_routes: capacity %d invalid", capacity);
    EVAMX_REQUIRE(rows >= 1 && rows <= capacity, "evamx_prepare_routes: rows %d outside 1..capacity", rows);
    EVAMX_REQUIRE(n_local >= 1 && n_local <= EVAMX_MAX_EXPERTS, "evamx_prepare_routes: n_local %d outside 1..%d",
                  n_local, EVAMX_MAX_EXPERTS);
    const size_t need = evamx_prepare_routes_workspace_bytes(capacity, topk);
    if (workspace_bytes < need) {
        set_error("evamx_prepare_routes: workspace %zu bytes < %zu", workspace_bytes, need);
        return EVAMX_ENOSPACE;
    }
    MoeParams p;
    memset(&p, 0, sizeof p);
    p.mode = PREP_GROUP;
    p.T = rows; p.topk = topk; p.n_local = n_local;
    p.sel = const_cast<int64_t*>(sel);
    p.rw16 = (half_t*)const_cast<void*>(rw_fp16);
    p.min_expert = -1;
    p.err = (int*)workspace;
    p.local = (int*)((char*)workspace + 256);
    p.runs = runs;
    p.slots_max = capacity * topk;
    moe_prepare_only(p, (hipStream_t)stream);
    return launched("prepare_routes");
}

extern "C" size_t evamx_moe_workspace_bytes(const evamx_moe_shape* shape)
{
    if (!shape_ok(shape)) return 0;
    return moe_layout(shape).total;
}

extern "C" float* evamx_moe_logits_ptr(const evamx_moe_shape* shape, void* workspace)
{
    if (!shape_ok(shape) || !workspace) return nullptr;
    return (float*)((char*)workspace + moe_layout(shape).logits);
}

extern "C" const void* evamx_moe_rotated_ptr(const evamx_moe_shape* shape, void* workspace)
{
    if (!shape_ok(shape) || !workspace) return nullptr;
    return (const void*)((char*)workspace + moe_layout(shape).xr);
}

extern "C" int32_t* evamx_moe_runs_ptr(const evamx_moe_shape* shape, void* workspace)
{
    if (!shape_ok(shape) || !workspace) return nullptr;
    return (int32_t*)((char*)workspace + moe_layout(shape).runs);
}

extern "C" int32_t* evamx_moe_flags_ptr(const evamx_moe_shape* shape, void* workspace)
{
    if (!shape_ok(shape) || !workspace) return nullptr;
    return (int32_t*)((char*)workspace + moe_layout(shape).flags);
}

extern "C" int evamx_moe_workspace_init(const evamx_moe_shape* shape, void* workspace, evamx_stream_t stream)
{
    g_err[0] = 0;
    if (!shape_ok(shape)) return EVAMX_EINVAL;
    EVAMX_REQUIRE(workspace, "evamx_moe_workspace_init: null workspace");
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (int*)((char*)workspace + moe_layout(shape).flags), 64, 0);
    return launched("workspace_init");
}

extern "C" int evamx_moe_forward(const evamx_moe_args* a, evamx_stream_t stream)
{
    g_err[0] = 0;
    EVAMX_REQUIRE(a, "evamx_moe_forward: null args");
    return moe_forward_ws(a, a->workspace, a->workspace_bytes, (hipStream_t)stream, "evamx_moe_forward", true);
}

size_t evamx::moe_workspace_bytes_of(const evamx_moe_shape* shape)
{
    return shape_ok(shape) ? moe_layout(shape).total : 0;
}

int evamx::moe_flags_offset(const evamx_moe_shape* shape, size_t* off)
{
    if (!shape_ok(shape)) return EVAMX_EINVAL;
    *off = moe_layout(shape).flags;
    return EVAMX_OK;
}

int evamx::moe_forward_ws(const evamx_moe_args* a, void* workspace, size_t workspace_bytes, hipStream_t stream,
                          const char* who, bool side_stream_ok)
{
    const evamx_moe_shape* s = &a->shape;
    if (!shape_ok(s)) return EVAMX_EINVAL;
    const MoeLayout L = moe_layout(s);
    EVAMX_REQUIRE(a->rows >= 1 && a->rows <= s->rows_max, "%s: rows %d outside 1..%d", who, a->rows, s->rows_max);
    EVAMX_REQUIRE(a->x && (a->out || a->residual) && a->tables && a->sel && workspace, "%s: null pointer", who);
    EVAMX_REQUIRE(a->x_dtype == EVAMX_DTYPE_F16 || a->x_dtype == EVAMX_DTYPE_BF16, "%s: x_dtype %d", who, a->x_dtype);
    EVAMX_REQUIRE(((uintptr_t)a->x & 3) == 0 && a->x_stride % 2 == 0,
                  "%s: x must be 4-byte aligned with an even row stride", who);
    EVAMX_REQUIRE(a->x_stride >= s->hidden && (!a->out || a->out_stride >= s->hidden) &&
                      (!a->residual || a->residual_stride >= s->hidden),
                  "%s: row strides below hidden", who);
    EVAMX_REQUIRE(std::isfinite(a->limit) && a->limit >= 0.0f, "%s: limit must be finite and >= 0", who);
    EVAMX_REQUIRE(!(a->logits && a->gate_w), "%s: give logits or gate_w, not both", who);
    EVAMX_REQUIRE(((uintptr_t)a->gate_w & 15) == 0, "%s: gate_w must be 16-byte aligned", who);
    if (a->logits || a->gate_w) {
        EVAMX_REQUIRE(a->n_logits >= s->topk && a->n_logits <= EVAMX_MAX_EXPERTS,
                      "%s: n_logits %d must be in topk..%d", who, a->n_logits, EVAMX_MAX_EXPERTS);
        EVAMX_REQUIRE(a->weights, "%s: routing needs a weights output", who);
        EVAMX_REQUIRE(a->score_fn == EVAMX_SCORE_SIGMOID || a->score_fn == EVAMX_SCORE_SQRT_SOFTPLUS,
                      "%s: unknown score function %d", who, a->score_fn);
        EVAMX_REQUIRE(std::isfinite(a->route_scale), "%s: route_scale must be finite", who);
    } else {
        EVAMX_REQUIRE(a->weights || a->rw_fp16, "%s: routes need fp32 weights or fp16 rw", who);
    }
    if (a->min_expert >= 0)
        EVAMX_REQUIRE(a->max_expert > a->min_expert, "%s: empty expert range", who);
    int k2u = 0;
    if (!a->k2_per_expert) {
        k2u = rate_k2(a->bits);
        EVAMX_REQUIRE(gemv_rate(k2u), "%s: bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", who, (double)a->bits);
    }
    int k2du = 0;                  // 0: the down rate follows the gate/up rate
    if (!a->k2_down_per_expert && a->bits_down != 0.0f) {
        k2du = rate_k2(a->bits_down);
        EVAMX_REQUIRE(gemv_rate(k2du), "%s: down bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", who, (double)a->bits_down);
    }
    int k2s = 0, k2sd = 0;
    if (s->has_shared) {
        EVAMX_REQUIRE(a->shared, "%s: shape has a shared expert but no pointers were given", who);
        for (int i = 0; i < 9; ++i) EVAMX_REQUIRE(a->shared[i] != 0, "%s: shared pointer %d is null", who, i);
        k2s = rate_k2(a->shared_bits);
        EVAMX_REQUIRE(gemv_rate(k2s), "%s: shared bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", who, (double)a->shared_bits);
        k2sd = k2s;
        if (a->shared_bits_down != 0.0f) {
            k2sd = rate_k2(a->shared_bits_down);
            EVAMX_REQUIRE(gemv_rate(k2sd), "%s: shared down bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", who,
                          (double)a->shared_bits_down);
        }
    }
    EVAMX_REQUIRE(!a->shared_gate_w || s->has_shared, "%s: shared_gate_w without a shared expert", who);
    EVAMX_REQUIRE(((uintptr_t)a->shared_gate_w & 3) == 0, "%s: shared_gate_w must be 4-byte aligned", who);
    if (workspace_bytes < L.total) {
        set_error("%s: workspace %zu bytes < %zu", who, workspace_bytes, L.total);
        return EVAMX_ENOSPACE;
    }

    char* ws = (char*)workspace;
    MoeParams p;
    memset(&p, 0, sizeof p);
    p.mode = PREP_GROUP | PREP_MOE;
    p.T = a->rows; p.H = s->hidden; p.I = s->inter; p.topk = s->topk; p.n_local = s->n_local;
    p.n_logits = a->n_logits;
    p.x = a->x; p.x_dtype = a->x_dtype; p.x_stride = a->x_stride;
    p.logits = a->logits; p.sel_bias = a->sel_bias; p.score = a->score_fn; p.route_scale = a->route_scale;
    p.gate_w = a->gate_w;
    if (a->gate_w) p.logits = (const float*)(ws + L.logits);     // written by the gate kernel
    p.sel = a->sel;
    p.weights = a->weights;
    p.rw16 = a->rw_fp16 ? (half_t*)a->rw_fp16 : (half_t*)(ws + L.rw16);
    if (!a->logits && !a->gate_w && !a->weights) p.weights = nullptr;    // rw_fp16 is the input
    p.min_expert = a->min_expert >= 0 ? a->min_expert : -1;
    p.max_expert = a->max_expert;
    p.tables = a->tables; p.tbl_stride = s->n_local;
    p.k2_per_expert = a->k2_per_expert; p.k2_uniform = k2u; p.k2_shared = k2s;
    p.k2d_per_expert = a->k2_down_per_expert; p.k2d_uniform = k2du; p.k2_shared_d = k2sd;
    p.sh_gate_w = (const half_t*)a->shared_gate_w;
    p.gate_val = (float*)(ws + L.gate_val);
    p.has_shared = s->has_shared ? 1 : 0;
    if (s->has_shared)
        for (int i = 0; i < 9; ++i) p.sh_ptr[i] = a->shared[i];
    p.limit = a->limit;
    p.err = (int*)(ws + L.flags);
    p.meta = (int*)(ws + L.meta);
    p.local = (int*)(ws + L.local);
    p.order = (int*)(ws + L.order);
    p.runs = (int*)(ws + L.runs);
    p.slots_max = L.slots_max;
    p.chunks = (int*)(ws + L.chunks);
    p.unit_chunk = (int*)(ws + L.unit_chunk);
    p.tiles = (int*)(ws + L.tiles);
    p.slot_mult = (int*)(ws + L.slot_mult);
    p.urec = (UnitRec*)(ws + L.urec);
    p.srec = (SlotRec*)(ws + L.srec);
    p.max_chunks = L.max_chunks;
    p.xr = (half_t*)(ws + L.xr);
    p.xsum = (float*)(ws + L.xsum);
    p.act = (half_t*)(ws + L.act);
    p.actsum = (float*)(ws + L.actsum);
    p.part_gu = (float*)(ws + L.part_gu);
    p.part_d = (float*)(ws + L.part_d);
    p.nslot_max = L.nslot_max;
    p.ks_gu = L.ks_gu; p.ks_d = L.ks_d;
    p.ks_gu_max = L.ks_gu_max; p.ks_d_max = L.ks_d_max;
    p.cap_rows_gu = L.cap_rows_gu; p.cap_rows_d = L.cap_rows_d;
    p.strict_rows = s->strict_rows;
    p.strict_ks_gu = L.strict_ks_gu; p.strict_ks_d = L.strict_ks_d;
    p.gemv_waves = gemv_waves();
    p.side_ok = side_stream_ok ? 1 : 0;
    p.out = a->out; p.out_stride = a->out_stride;
    p.residual = (uint16_t*)a->residual; p.residual_stride = a->residual_stride;
    moe_launch(p, stream, a->events);
    return launched(who);
}

extern "C" int evamx_bench_decode(float bits, int waves, int iters, float* sink, evamx_stream_t stream)
{
    g_err[0] = 0;
    const int k2 = rate_k2(bits);
    EVAMX_REQUIRE(sink, "evamx_bench_decode: null sink");
    EVAMX_REQUIRE(gemv_rate(k2), "evamx_bench_decode: bit rate %g not in {1.5,2,2.5,3,3.5,4,5}", (double)bits);
    EVAMX_REQUIRE(waves >= 4 && waves <= (1 << 22) && waves % 4 == 0, "evamx_bench_decode: waves %d not a multiple of 4 in 4..%d",
                  waves, 1 << 22);
    EVAMX_REQUIRE(iters >= 1 && iters <= (1 << 20), "evamx_bench_decode: iters %d outside 1..%d", iters, 1 << 20);
    launch_bench_decode(k2, waves / 4, iters, sink, (hipStream_t)stream);
    return launched("bench_decode");
}

extern "C" int evamx_bench_read(const void* buf, size_t bytes, int ncg, int rows, int waves, float* sink,
                                evamx_stream_t stream)
{
    g_err[0] = 0;
    EVAMX_REQUIRE(buf && sink, "evamx_bench_read: null buffer or sink");
    EVAMX_REQUIRE(ncg >= 1 && ncg <= 4096, "evamx_bench_read: ncg %d outside 1..4096", ncg);
    EVAMX_REQUIRE(rows >= 1 && rows <= (1 << 20), "evamx_bench_read: rows %d outside 1..%d", rows, 1 << 20);
    EVAMX_REQUIRE(waves >= ncg && waves <= (1 << 22) && waves % ncg == 0,
                  "evamx_bench_read: waves %d not a multiple of ncg %d in %d..%d", waves, ncg, ncg, 1 << 22);
    const double need = (double)(waves / ncg) * rows * ncg * 1024.0;
    EVAMX_REQUIRE(need <= (double)bytes, "evamx_bench_read: the shape reads %.0f bytes, the buffer holds %zu", need, bytes);
    launch_bench_read(buf, ncg, rows, waves, sink, (hipStream_t)stream);
    return launched("bench_read");
}
