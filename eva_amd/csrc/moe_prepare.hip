// Prepare stage of the decode-shaped MoE pipeline (routing, slot activity, stable grouping,
// records or chunks, input rotations) and the router front: the kernels and their launches.
// The launch sequence is in moe_decode.hip.
#include "moe_common.hpp"

namespace evamx {

__global__ __launch_bounds__(256) void moe_gate_kernel(MoeParams p, float* logits)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    const int ngr = (p.T + GATE_ROWS - 1) / GATE_ROWS;
    if (wid >= p.n_logits * ngr) return;
    const int e = wid / ngr, r0 = (wid - e * ngr) * GATE_ROWS;
    const float4* w = (const float4*)(p.gate_w + (size_t)e * p.H);
    float acc[GATE_ROWS];
#pragma unroll
    for (int r = 0; r < GATE_ROWS; ++r) acc[r] = 0.0f;
    for (int k4 = lane; k4 < p.H / 4; k4 += 64) {
        const float4 wv = w[k4];
#pragma unroll
        for (int r = 0; r < GATE_ROWS; ++r) {
            if (r0 + r < p.T) {
                const int k = 4 * k4;
                float a = acc[r];
                a = fmaf(x_at(p, r0 + r, k + 0), wv.x, a);
                a = fmaf(x_at(p, r0 + r, k + 1), wv.y, a);
                a = fmaf(x_at(p, r0 + r, k + 2), wv.z, a);
                a = fmaf(x_at(p, r0 + r, k + 3), wv.w, a);
                acc[r] = a;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GATE_ROWS; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && r0 + r < p.T) logits[(size_t)(r0 + r) * p.n_logits + e] = v;
    }
}

// ---------------------------------------------------------------------------------------------
// Prepare for small batches (T*topk <= EVAMX_SMALL_SLOTS, T <= EVAMX_SMALL_ROWS): every
// workgroup routes in LDS, one wave per token (workgroups of max(4, T) waves); workgroup 0
// groups the slots and publishes the tables while the others rotate the active slots' inputs
// (rotations are stored by slot, so they need no order).


struct SmallLds {
    ExpertLds ex;
    int sel[EVAMX_SMALL_SLOTS];
    half_t rw[EVAMX_SMALL_SLOTS];
    int local[EVAMX_SMALL_SLOTS];
    int order[EVAMX_SMALL_SLOTS + EVAMX_SMALL_ROWS];
};

__global__ __launch_bounds__(64 * EVAMX_SMALL_ROWS) void moe_prepare_small_kernel(MoeParams p)
{
    __shared__ SmallLds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nt = blockDim.x, nwv = nt >> 6;
    const int slots = p.T * p.topk;
    const bool pub = blockIdx.x == 0;
    if (p.logits) {
        for (int r = wave; r < p.T; r += nwv) route_token(p, r, lane, sh.sel, sh.rw, pub);
    } else {
        for (int s = t; s < slots; s += nt) {
            const int64_t e = p.sel[s];
            // indices outside the int range are outside any table: keep them out of range
            sh.sel[s] = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
            sh.rw[s] = p.weights ? f2h(p.weights[s]) : p.rw16[s];
            if (pub && p.weights) p.rw16[s] = sh.rw[s];
        }
    }
    if (pub && p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += nt) p.runs[i] = 0;
    }
    __syncthreads();
    if (!pub) {
        // rotation workgroups need only each slot's expert: the grouping is workgroup 0's
        for (int s = t; s < slots; s += nt) sh.local[s] = slot_local(p, sh.sel[s], sh.rw[s], false);
        __syncthreads();
        rotate_rows(p, nullptr, sh.local, slots + (p.has_shared ? p.T : 0), (blockIdx.x - 1) * nwv + wave,
                    (gridDim.x - 1) * nwv, lane);
        return;
    }
    group_slots(p, sh.sel, sh.rw, slots, sh.local, sh.order, sh.ex, pub);
    const int n_active = sh.ex.off[p.n_local];
    if (p.has_shared)
        for (int r = t; r < p.T; r += nt) sh.order[n_active + r] = slots + r;
    __syncthreads();
    {
        for (int s = t; s < slots; s += nt) p.local[s] = sh.local[s];
        for (int i = t; i < n_active + (p.has_shared ? p.T : 0); i += nt) p.order[i] = sh.order[i];
        write_chunks(p, sh.ex, sh.order);
        if (t == 0) {
            p.runs[0] = sh.ex.run_base[p.n_local];
            p.runs[1] = 0;
            p.runs[2 + sh.ex.run_base[p.n_local]] = n_active;
            p.meta[0] = total_chunks(p, sh.ex);
            p.meta[1] = n_active;
            p.meta[2] = total_units(p, sh.ex);
        }
    }
}

// Prepare of the decode path (calls of at most EVAMX_GEMV_MAX_ROWS rows, so at most 64 slots):
// waves [0, T) route one token each while the other waves copy the [9][n_local] pointer table
// (and the per-expert rates) into LDS; then wave 0 alone groups the slots with one key per lane
// sorted across the wave (key (local expert, slot): the stable order by expert), cuts runs of at
// most EVAMX_CHUNK slots at expert changes (the reference run table's runs, which are also the
// GEMV chunks), and writes the run table and the unit and slot records from registers and LDS.
constexpr int GEMV_PREP_WAVES = 4;

struct GemvPrepLds {
    uint64_t tbl[9][EVAMX_MAX_EXPERTS];
    uint8_t k2[EVAMX_MAX_EXPERTS];
    uint8_t k2d[EVAMX_MAX_EXPERTS];
    int sel[64];
    half_t rw[64];
};

__global__ __launch_bounds__(64 * GEMV_PREP_WAVES) void moe_prepare_gemv_kernel(MoeParams p)
{
    __shared__ GemvPrepLds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int slots = p.T * p.topk;               // at most 2 * EVAMX_MAX_TOPK = 64
    const int E = p.n_local;
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += blockDim.x) p.runs[i] = 0;
    }
    if (wave < p.T) {
        if (p.logits) route_token(p, wave, lane, sh.sel, sh.rw, true);      // writes slots wave * topk + j
    } else {
        const int nt = (GEMV_PREP_WAVES - p.T) * 64, i0 = t - p.T * 64;
        for (int i = i0; i < 9 * E; i += nt) sh.tbl[i / E][i % E] = (uint64_t)p.tables[(size_t)(i / E) * p.tbl_stride + i % E];
        for (int i = i0; i < E; i += nt) {
            sh.k2[i] = (uint8_t)k2_gu_of(p, i);
            sh.k2d[i] = (uint8_t)k2_d_of(p, i);
        }
    }
    if (!p.logits && t < slots) {
        const int64_t e = p.sel[t];
        sh.sel[t] = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
        sh.rw[t] = p.weights ? f2h(p.weights[t]) : p.rw16[t];
        if (p.weights) p.rw16[t] = sh.rw[t];
    }
    __syncthreads();
    if (wave != 0) return;

    // slot activity (lane = slot), the published local expert, inactive slot records
    int e = -1;
    if (lane < slots) {
        e = slot_local(p, sh.sel[lane], sh.rw[lane], true);
        p.local[lane] = e;
        if (e < 0) {
            SlotRec q = {};
            p.srec[lane] = q;
        }
    }
    // stable grouping: sort keys (expert, slot); inactive slots sort last
    const uint32_t key = wave_sort_asc(e >= 0 ? ((uint32_t)e << 6) | (uint32_t)lane : 0xffffffffu, lane);
    const bool act = key != 0xffffffffu;
    const int ge = (int)(key >> 6), gs = (int)(key & 63);
    const uint64_t amask = __ballot(act);
    const int n_active = __popcll(amask);
    const int prev_e = __shfl_up(ge, 1, WAVE);
    const uint64_t heads = __ballot(act && (lane == 0 || prev_e != ge));
    const uint64_t le_mask = lane == 63 ? ~0ull : ((2ull << lane) - 1);     // lanes 0..lane
    const int first = 63 - __clzll(heads & le_mask);                        // the expert's first position
    const bool rs = act && ((lane - first) % EVAMX_CHUNK) == 0;             // run (chunk) start
    const uint64_t rmask = __ballot(rs);
    const int n_runs = __popcll(rmask);
    const uint64_t above = rmask & ~le_mask;
    const int next = above ? __ffsll((long long)above) - 1 : n_active;
    const int rows = rs ? next - lane : 0;
    const int m = rs ? unit_mult(p, rows) : 0;
    const int m_incl = wave_incl_scan(m);
    const int ubase = m_incl - m;
    const int routed_units = __builtin_amdgcn_readlane(m_incl, 63);
    const KSplit kgu = ks_gate_up(p, p.units_max), kd = ks_down(p, p.units_max);
    // the chunk of each position: its run start's lane
    const int rlane = act ? 63 - __clzll(rmask & le_mask) : 0;
    const int my_m = __shfl(m, rlane, WAVE);
    int slot_run[EVAMX_CHUNK];
#pragma unroll
    for (int j = 0; j < EVAMX_CHUNK; ++j) slot_run[j] = __shfl(gs, lane + j < 64 ? lane + j : 63, WAVE);

    if (act) {
        // run table (moe_coop3072.py:86-106): order, run starts
        if (p.runs) {
            p.runs[2 + p.slots_max + 1 + lane] = gs;
            if (rs) p.runs[2 + __popcll(rmask & (le_mask >> 1)) ] = lane;
        }
        p.order[lane] = gs;
        const int k2 = sh.k2[ge], k2d = sh.k2d[ge];
        SlotRec q;
        q.active = 1;
        q.shared = 0;
        q.s_gu = ks_of_chunk(kgu, my_m);
        q.s_d = ks_of_chunk(kd, my_m);
        q.w = h2f(sh.rw[gs]);
        q.pad[0] = q.pad[1] = q.pad[2] = 0;
        q.g_svh = sh.tbl[EVAMX_TBL_G_SVH][ge];
        q.u_svh = sh.tbl[EVAMX_TBL_U_SVH][ge];
        q.d_suh = sh.tbl[EVAMX_TBL_D_SUH][ge];
        q.d_svh = sh.tbl[EVAMX_TBL_D_SVH][ge];
        p.srec[gs] = q;
        if (rs) {
            if (!gemv_k2_supported(k2) || !gemv_k2_supported(k2d)) atomicOr(p.err, EVAMX_ERR_RATE);
            UnitRec r;
            r.e = ge;
            r.rows = rows;
            r.k2 = k2;
            r.ubase = ubase;
            r.s_gu = ks_of_chunk(kgu, m);
            r.s_d = ks_of_chunk(kd, m);
            r.k2_d = k2d;
            r.pair = 0;
#pragma unroll
            for (int j = 0; j < EVAMX_CHUNK; ++j) r.slot[j] = j < rows ? slot_run[j] : slot_run[0];
            r.tr[0] = sh.tbl[EVAMX_TBL_G_TRELLIS][ge];
            r.tr[1] = sh.tbl[EVAMX_TBL_U_TRELLIS][ge];
            r.tr[2] = sh.tbl[EVAMX_TBL_D_TRELLIS][ge];
            r.suh[0] = sh.tbl[EVAMX_TBL_G_SUH][ge];
            r.suh[1] = sh.tbl[EVAMX_TBL_U_SUH][ge];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            for (int i = 0; i < m; ++i) p.urec[ubase + i] = r;
        }
    }
    // the shared expert: one chunk of the T rows after the routed ones
    int n_units = routed_units;
    if (p.has_shared) {
        if (lane < p.T) {
            p.order[n_active + lane] = slots + lane;
            SlotRec q;
            q.active = 1;
            q.shared = 1;
            q.s_gu = ks_of_chunk(kgu, 1);
            q.s_d = ks_of_chunk(kd, 1);
            q.w = 1.0f;
            q.pad[0] = q.pad[1] = q.pad[2] = 0;
            q.g_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SVH];
            q.u_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SVH];
            q.d_suh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SUH];
            q.d_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SVH];
            p.srec[slots + lane] = q;
        }
        if (lane == 0) {
            UnitRec r;
            r.e = -1;
            r.rows = p.T;
            r.k2 = p.k2_shared;
            r.ubase = routed_units;
            r.s_gu = ks_of_chunk(kgu, 1);
            r.s_d = ks_of_chunk(kd, 1);
            r.k2_d = p.k2_shared_d;
            r.pair = 0;
#pragma unroll
            for (int j = 0; j < EVAMX_CHUNK; ++j) r.slot[j] = slots + (j < p.T ? j : 0);
            r.tr[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_TRELLIS];
            r.tr[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_TRELLIS];
            r.tr[2] = (uint64_t)p.sh_ptr[EVAMX_TBL_D_TRELLIS];
            r.suh[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SUH];
            r.suh[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SUH];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            p.urec[routed_units] = r;
        }
        n_units += 1;      // T <= 2 rows: one chunk of weight 1
    }
    for (int u = n_units + lane; u < p.units_max; u += 64) p.urec[u].e = EVAMX_NO_UNIT;
    if (lane == 0) {
        if (p.runs) {
            p.runs[0] = n_runs;
            p.runs[1] = 0;
            p.runs[2 + n_runs] = n_active;
        }
        p.meta[0] = n_runs + (p.has_shared ? 1 : 0);
        p.meta[1] = n_active;
        p.meta[2] = n_units;
        p.meta[3] = 0;
    }
}

// Prepare of the decode path for calls of 3 or more rows (strict mode, at most
// EVAMX_STRICT_MAX_SLOTS slots): one workgroup of WIDE_PREP_WAVES waves. Up to 12 waves route the
// tokens (a wave per token at a time) while the others copy the pointer table and the rates into
// LDS; the workgroup then groups the slots stably by (expert, slot) into LDS (group_slots, which
// also publishes the run table), and every thread writes the records of some grouped positions:
// the slot record of each active slot and, at each chunk start (every EVAMX_CHUNK positions of an
// expert), the unit record(s) of that chunk. The shared expert's rows follow as chunks of
// EVAMX_CHUNK rows. The same records, splits and order as moe_prepare_gemv_kernel would write.
constexpr int WIDE_PREP_WAVES = 16;

struct WidePrepLds {
    uint64_t tbl[9][EVAMX_MAX_EXPERTS];
    uint8_t k2[EVAMX_MAX_EXPERTS];
    uint8_t k2d[EVAMX_MAX_EXPERTS];
    int sel[EVAMX_STRICT_MAX_SLOTS];
    half_t rw[EVAMX_STRICT_MAX_SLOTS];
    int local[EVAMX_STRICT_MAX_SLOTS];
    int order[EVAMX_STRICT_MAX_SLOTS];
    ExpertLds ex;
};

__global__ __launch_bounds__(64 * WIDE_PREP_WAVES) void moe_prepare_wide_kernel(MoeParams p)
{
    __shared__ WidePrepLds sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nt = blockDim.x;
    const int slots = p.T * p.topk;               // at most EVAMX_STRICT_MAX_SLOTS (checked on the host)
    const int E = p.n_local;
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += nt) p.runs[i] = 0;
    }
    const int nrw = p.logits ? min(p.T, WIDE_PREP_WAVES - 4) : 0;
    if (wave < nrw) {
        for (int r = wave; r < p.T; r += nrw) route_token(p, r, lane, sh.sel, sh.rw, true);
    } else {
        const int nc = (WIDE_PREP_WAVES - nrw) * 64, i0 = t - nrw * 64;
        for (int i = i0; i < 9 * E; i += nc) sh.tbl[i / E][i % E] = (uint64_t)p.tables[(size_t)(i / E) * p.tbl_stride + i % E];
        for (int i = i0; i < E; i += nc) {
            sh.k2[i] = (uint8_t)k2_gu_of(p, i);
            sh.k2d[i] = (uint8_t)k2_d_of(p, i);
        }
    }
    if (!p.logits) {
        for (int s = t; s < slots; s += nt) {
            const int64_t e = p.sel[s];
            sh.sel[s] = (e >= 0 && e < 0x7fffffff) ? (int)e : -1;
            sh.rw[s] = p.weights ? f2h(p.weights[s]) : p.rw16[s];
            if (p.weights) p.rw16[s] = sh.rw[s];
        }
    }
    __syncthreads();
    // slot activity, stable order by (expert, slot), run table entries, per-expert offsets
    group_slots(p, sh.sel, sh.rw, slots, sh.local, sh.order, sh.ex, true);
    const ExpertLds& ex = sh.ex;
    const int n_active = ex.off[E];
    const int routed_units = ex.unit_base[E];
    // units longest first: the shared expert's (its chunks carry every row of the call), then the
    // routed experts' by row count (unit_order_base), so that the GEMV launches start their
    // longest waves first and their last round holds short ones
    const int sh_units = p.has_shared ? expert_units(p, p.T) : 0;
    const KSplit kgu = ks_gate_up(p, p.units_max), kd = ks_down(p, p.units_max);
    for (int s = t; s < slots; s += nt) {
        const int e = sh.local[s];
        p.local[s] = e;
        if (e < 0) {
            SlotRec q = {};
            p.srec[s] = q;
        }
    }
    for (int pos = t; pos < n_active; pos += nt) {
        const int s = sh.order[pos];
        const int e = sh.local[s];
        const int j = pos - ex.off[e];             // rank within the expert's slots
        const int c = j / EVAMX_CHUNK;             // the expert's chunk
        const int rows = min(EVAMX_CHUNK, ex.cnt[e] - c * EVAMX_CHUNK);
        const int m = unit_mult(p, rows);
        p.order[pos] = s;
        SlotRec q;
        q.active = 1;
        q.shared = 0;
        q.s_gu = ks_of_chunk(kgu, m);
        q.s_d = ks_of_chunk(kd, m);
        q.w = h2f(sh.rw[s]);
        q.pad[0] = q.pad[1] = q.pad[2] = 0;
        q.g_svh = sh.tbl[EVAMX_TBL_G_SVH][e];
        q.u_svh = sh.tbl[EVAMX_TBL_U_SVH][e];
        q.d_suh = sh.tbl[EVAMX_TBL_D_SUH][e];
        q.d_svh = sh.tbl[EVAMX_TBL_D_SVH][e];
        p.srec[s] = q;
        if (j % EVAMX_CHUNK == 0) {
            const int k2 = sh.k2[e], k2d = sh.k2d[e];
            if (!gemv_k2_supported(k2) || !gemv_k2_supported(k2d)) atomicOr(p.err, EVAMX_ERR_RATE);
            const int ubase = sh_units + unit_order_base(ex, E, e) + c * unit_mult(p, EVAMX_CHUNK);    // earlier chunks are full
            UnitRec r;
            r.e = e;
            r.rows = rows;
            r.k2 = k2;
            r.ubase = ubase;
            r.s_gu = q.s_gu;
            r.s_d = q.s_d;
            r.k2_d = k2d;
            r.pair = pair_units(p) ? unit_pair(c, (ex.cnt[e] + EVAMX_CHUNK - 1) / EVAMX_CHUNK) : 0;
#pragma unroll
            for (int i = 0; i < EVAMX_CHUNK; ++i) r.slot[i] = sh.order[pos + (i < rows ? i : 0)];
            r.tr[0] = sh.tbl[EVAMX_TBL_G_TRELLIS][e];
            r.tr[1] = sh.tbl[EVAMX_TBL_U_TRELLIS][e];
            r.tr[2] = sh.tbl[EVAMX_TBL_D_TRELLIS][e];
            r.suh[0] = sh.tbl[EVAMX_TBL_G_SUH][e];
            r.suh[1] = sh.tbl[EVAMX_TBL_U_SUH][e];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            for (int i = 0; i < m; ++i) p.urec[ubase + i] = r;
        }
    }
    // the shared expert: chunks of EVAMX_CHUNK of its T rows, units [0, sh_units)
    const int n_units = routed_units + sh_units;
    if (p.has_shared) {
        const int nsc = (p.T + EVAMX_CHUNK - 1) / EVAMX_CHUNK;
        for (int r = t; r < p.T; r += nt) {
            const int rows = min(EVAMX_CHUNK, p.T - (r / EVAMX_CHUNK) * EVAMX_CHUNK);
            const int m = unit_mult(p, rows);
            p.order[n_active + r] = slots + r;
            SlotRec q;
            q.active = 1;
            q.shared = 1;
            q.s_gu = ks_of_chunk(kgu, m);
            q.s_d = ks_of_chunk(kd, m);
            q.w = 1.0f;
            q.pad[0] = q.pad[1] = q.pad[2] = 0;
            q.g_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SVH];
            q.u_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SVH];
            q.d_suh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SUH];
            q.d_svh = (uint64_t)p.sh_ptr[EVAMX_TBL_D_SVH];
            p.srec[slots + r] = q;
        }
        for (int c = t; c < nsc; c += nt) {
            const int rows = min(EVAMX_CHUNK, p.T - c * EVAMX_CHUNK);
            const int m = unit_mult(p, rows);
            const int ubase = c * unit_mult(p, EVAMX_CHUNK);
            UnitRec r;
            r.e = -1;
            r.rows = rows;
            r.k2 = p.k2_shared;
            r.ubase = ubase;
            r.s_gu = ks_of_chunk(kgu, m);
            r.s_d = ks_of_chunk(kd, m);
            r.k2_d = p.k2_shared_d;
            r.pair = pair_units(p) ? unit_pair(c, nsc) : 0;
#pragma unroll
            for (int i = 0; i < EVAMX_CHUNK; ++i) r.slot[i] = slots + c * EVAMX_CHUNK + (i < rows ? i : 0);
            r.tr[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_TRELLIS];
            r.tr[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_TRELLIS];
            r.tr[2] = (uint64_t)p.sh_ptr[EVAMX_TBL_D_TRELLIS];
            r.suh[0] = (uint64_t)p.sh_ptr[EVAMX_TBL_G_SUH];
            r.suh[1] = (uint64_t)p.sh_ptr[EVAMX_TBL_U_SUH];
            r.pad1[0] = r.pad1[1] = r.pad1[2] = 0;
            for (int i = 0; i < m; ++i) p.urec[ubase + i] = r;
        }
    }
    for (int u = n_units + t; u < p.units_max; u += nt) p.urec[u].e = EVAMX_NO_UNIT;
    if (t == 0) {
        const int n_runs = ex.run_base[E];
        if (p.runs) {
            p.runs[0] = n_runs;
            p.runs[1] = 0;
            p.runs[2 + n_runs] = n_active;
        }
        p.meta[0] = n_runs + (p.has_shared ? (p.T + EVAMX_CHUNK - 1) / EVAMX_CHUNK : 0);
        p.meta[1] = n_active;
        p.meta[2] = n_units;
        p.meta[3] = 0;
    }
}

// ---------------------------------------------------------------------------------------------
// Prepare for any batch, in three launches: routing (one wave per token), grouping (one
// workgroup of 1024 threads, per-slot arrays in global memory), rotations (a full grid).

__global__ __launch_bounds__(256) void moe_route_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int r = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    if (r < p.T) route_token(p, r, lane, nullptr, nullptr, true);
}

__global__ __launch_bounds__(64 * GROUP_WAVES) void moe_group_kernel(MoeParams p)
{
    __shared__ ExpertLds ex;
    __shared__ GroupLds gl;
    const int t = threadIdx.x;
    const int slots = p.T * p.topk;
    if (!p.logits && p.weights)
        for (int s = t; s < slots; s += 1024) p.rw16[s] = f2h(p.weights[s]);
    if (p.runs) {
        const int table_len = 2 + 2 * p.slots_max + 1;
        for (int i = t; i < table_len; i += 1024) p.runs[i] = 0;
    }
    __syncthreads();
    group_slots_par(p, p.sel, p.rw16, slots, p.local, p.order, ex, gl, true);
    const int n_active = ex.off[p.n_local];
    if (t == 0 && p.runs) {
        p.runs[0] = ex.run_base[p.n_local];
        p.runs[1] = 0;
        p.runs[2 + ex.run_base[p.n_local]] = n_active;
    }
    if (!(p.mode & PREP_MOE)) return;
    if (p.has_shared)
        for (int r = t; r < p.T; r += 1024) p.order[n_active + r] = slots + r;
    __syncthreads();                 // the shared rows of the order are read by write_chunks
    write_chunks(p, ex, p.order);
    if (t == 0) {
        p.meta[0] = total_chunks(p, ex);
        p.meta[1] = n_active;
        p.meta[2] = total_units(p, ex);
    }
}

constexpr int EVAMX_ROTATE_BLOCKS = 2048;

__global__ __launch_bounds__(256) void moe_rotate_kernel(MoeParams p)
{
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    rotate_rows(p, p.order, p.local, p.meta[1] + (p.has_shared ? p.T : 0), w, gridDim.x * 4, lane);
}

// ---------------------------------------------------------------------------------------------
// Host side.

bool moe_small_path(int T, int topk) { return T * topk <= EVAMX_SMALL_SLOTS && T <= EVAMX_SMALL_ROWS; }

void launch_router_front(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const int waves = p.n_logits * ((p.T + GATE_ROWS - 1) / GATE_ROWS);
    launch_timed(moe_gate_kernel, dim3((waves + 3) / 4), dim3(256), stream, start, stop, p, const_cast<float*>(p.logits));
}

void launch_prepare(const MoeParams& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop)
{
    const int nch = p.H / 128;
    const int nslot = moe_nslot(p);
    if (!p.mfma) {
        // decode path: one workgroup routes, groups and writes the records; the gate/up waves
        // rotate their own inputs
        if (p.T <= EVAMX_GEMV_MAX_ROWS)
            launch_timed(moe_prepare_gemv_kernel, dim3(1), dim3(64 * GEMV_PREP_WAVES), stream, start, stop, p);
        else
            launch_timed(moe_prepare_wide_kernel, dim3(1), dim3(64 * WIDE_PREP_WAVES), stream, start, stop, p);
    } else if (moe_small_path(p.T, p.topk)) {
        // workgroup 0 groups, the others rotate; a wave per token routes in every workgroup
        // at most one workgroup per CU (gemv_waves = 16 per CU), so that none waits for a slot
        const int nwv = p.T > 4 ? p.T : 4;
        const int cus = p.gemv_waves / 16 > 2 ? p.gemv_waves / 16 : 2;
        int blocks = 1 + (nslot * nch * 2 + nwv - 1) / nwv;
        if (blocks > cus) blocks = cus;
        launch_timed(moe_prepare_small_kernel, dim3(blocks), dim3(64 * nwv), stream, start, stop, p);
    } else {
        if (p.logits) {
            launch_timed(moe_route_kernel, dim3((p.T + 3) / 4), dim3(256), stream, start, nullptr, p);
            start = nullptr;
        }
        launch_timed(moe_group_kernel, dim3(1), dim3(64 * GROUP_WAVES), stream, start, nullptr, p);
        launch_timed(moe_rotate_kernel, dim3(EVAMX_ROTATE_BLOCKS), dim3(256), stream, nullptr, stop, p);
    }
}

int moe_prepare_only(MoeParams& p, hipStream_t stream)
{
    if (p.logits) hipLaunchKernelGGL(moe_route_kernel, dim3((p.T + 3) / 4), dim3(256), 0, stream, p);
    if (p.mode & PREP_GROUP) hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(64 * GROUP_WAVES), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_router_logits(const MoeParams& p, float* logits, hipStream_t stream)
{
    const int waves = p.n_logits * ((p.T + GATE_ROWS - 1) / GATE_ROWS);
    hipLaunchKernelGGL(moe_gate_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p, logits);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
