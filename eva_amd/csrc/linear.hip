// Single EXL3 linear, fp16 in / fp16 out (the config-1 layer).
//
// Reference: ELinear.forward -> LinearEXL3 (runtime/ds41/exl3_linear.py:97-131), kernel
// exl3_gemv_kernel.cuh:217-234 (input: fp16 x*suh, Hadamard, fp16), 295-459 (GEMV, fp16 C),
// 463-490 with hadamard_inner.cuh:93-147 (output Hadamard to fp16, fp16 product with svh).
// Up to 2 rows, one launch: a k-split decode GEMV whose waves rotate their own input chunks
// (fp16(H128(fp16(x * suh)))) into LDS while their first weight loads are in flight, writing fp32
// partials; the workgroup that arrives last at its column group's counter then runs that group's
// output epilogue (the partials summed in fixed split order, fp16 C, Hadamard, fp16 svh product).
// 3 to 16 rows, three launches: the input rotation, the same GEMV on the rotated rows, and the
// same epilogue in a launch of its own.
// More rows, two launches: the input rotation, then the MFMA path, one workgroup per (64-row
// tile, 128 output columns) whose waves take fixed k-ranges, meet in LDS (summed in wave
// order) and run the output epilogue. In both paths a row's arithmetic depends on in/out only,
// not on how many rows share the call.
#include "evamx_internal.hpp"
#include "evamx_mfma.hpp"

namespace evamx {


__constant__ int k_iota64[64] = {0,  1,  2,  3,  4,  5,  6,  7,  8,  9,  10, 11, 12, 13, 14, 15,
                                 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31,
                                 32, 33, 34, 35, 36, 37, 38, 39, 40, 41, 42, 43, 44, 45, 46, 47,
                                 48, 49, 50, 51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61, 62, 63};

constexpr int LIN_GEMV_ROWS = 16;     // decode GEMV up to this many rows, MFMA tiles beyond
constexpr int LIN_ROT_ROWS = 2;       // the GEMV rotates its own inputs up to this many rows
// Weight prefetch depth of the 1-2 row GEMV: its waves stream 8 k-slices each at 2048 x 7168,
// one wave per SIMD; 3 slices in flight measured best (2: 7.58, 3: 6.84, 4: 6.98,
// 5: 7.07 us per call; the MoE's longer items keep 4).
constexpr int LIN_PF = 3;

struct LinParams {
    const half_t* x;
    int rows, in, out, k2, ks;
    const uint32_t* trellis;
    const half_t* suh;
    const half_t* svh;
    half_t* y;
    half_t* xr;        // [rows][in]
    float* xsum;       // [rows][in/128]
    float* part;       // [ks][rows][out]
    unsigned long long* arrive;   // arrival counters of the decode path, one per ARRIVE_STRIDE words
};

// Rotated inputs of tm rows (rows r0 .. r0 + tm - 1 of x) over the 128-chunks [w0, w1) into
// the wave's LDS rows (row m at dst + m * LIN_CW * 64 words, chunk w0 + j at word 64 j), with
// each row's chunk sums added in chunk order; the same operations as lin_rotate_kernel, so the
// rows are bit-identical to its output. issue() loads the x and suh words before the weight
// prefetch ring, finish() rotates them once the ring is in flight.
constexpr int LIN_CW = 4;             // 128-chunks per LDS window

template <int TM>
struct LinRot {
    static constexpr bool kWork = true;
    const LinParams& p;
    int tm, w0, w1, lane;
    __amdgpu_buffer_rsrc_t xrs[TM], srs;
    uint32_t* dst;
    float (&xs)[TM];
    uint32_t xv[TM][LIN_CW], sv[LIN_CW];

    __device__ __forceinline__ void issue()
    {
        // chunks past the window reload its last one (in bounds, unused): no branches
#pragma unroll
        for (int j = 0; j < LIN_CW; ++j)
            sv[j] = __builtin_amdgcn_raw_buffer_load_b32(srs, 4 * lane, 256 * min(w0 + j, w1 - 1), 0);
#pragma unroll
        for (int m = 0; m < TM; ++m)
#pragma unroll
            for (int j = 0; j < LIN_CW; ++j)
                xv[m][j] = __builtin_amdgcn_raw_buffer_load_b32(xrs[m], 4 * lane, 256 * min(w0 + j, w1 - 1), 0);
    }
    __device__ __forceinline__ void finish()
    {
#pragma unroll
        for (int m = 0; m < TM; ++m) {
            if (m >= tm) continue;
#pragma unroll
            for (int j = 0; j < LIN_CW; ++j) {
                if (w0 + j < w1) {
                    const half2_t xx = __builtin_bit_cast(half2_t, xv[m][j]);
                    const half2_t su = __builtin_bit_cast(half2_t, sv[j]);
                    float v0 = h2f(f2h(h2f(xx.x) * h2f(su.x)));      // fp16 product
                    float v1 = h2f(f2h(h2f(xx.y) * h2f(su.y)));
                    had128_pair(v0, v1, lane);
                    const half2_t r = {f2h(v0), f2h(v1)};
                    dst[m * LIN_CW * 64 + j * 64 + lane] = __builtin_bit_cast(uint32_t, r);
                    xs[m] += wave_sum(h2f(r.x) + h2f(r.y));
                }
            }
        }
        wave_lds_fence();
    }
};

template <int K2, int TM>
__device__ __forceinline__ void lin_rows(const LinParams& p, int r0, int tm, int cg, int ks, int c0, int c1, uint32_t* lds)
{
    const int lane = threadIdx.x & 63;
    __amdgpu_buffer_rsrc_t xrs[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) xrs[m] = weight_rsrc((const uint32_t*)(p.x + (size_t)(r0 + (m < tm ? m : 0)) * p.in));
    const __amdgpu_buffer_rsrc_t srs = weight_rsrc((const uint32_t*)p.suh);
    float acc[TM][2], xs[TM];
#pragma unroll
    for (int m = 0; m < TM; ++m) acc[m][0] = acc[m][1] = xs[m] = 0.0f;
    auto window = [&](int w0, int w1) {
        const XLds src{lds, LIN_CW * 64, 8 * w0};
        LinRot<TM> stage{p, tm, w0, w1, lane, {}, srs, lds, xs};
#pragma unroll
        for (int m = 0; m < TM; ++m) stage.xrs[m] = xrs[m];
        gemv_wave<K2, TM, LIN_PF>(p.trellis, p.out / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
    };
    if (c1 - c0 <= LIN_CW) {
        window(c0, c1);
    } else {
        for (int w0 = c0; w0 < c1; w0 += LIN_CW) {
            window(w0, min(c1, w0 + LIN_CW));
            wave_lds_fence();           // this window's reads before the next window's writes
        }
    }
    const int col0 = cg * 128 + lane_col(lane, 0), col1 = cg * 128 + lane_col(lane, 1);
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        if (m < tm) {
            float* dst = p.part + ((size_t)ks * p.rows + r0 + m) * p.out;
            store_wt(dst + col0, mul1_affine(acc[m][0], xs[m]));
            store_wt(dst + col1, mul1_affine(acc[m][1], xs[m]));
        }
    }
}

template <int K2, int TM>
__device__ __forceinline__ void lin_item(const LinParams& p, int cg, int ks, int c0, int c1, uint32_t* lds)
{
    if constexpr (TM == 1) lin_rows<K2, 1>(p, 0, 1, cg, ks, c0, c1, lds);
    else lin_rows<K2, 2>(p, 0, p.rows, cg, ks, c0, c1, lds);
}

// Partials of 16 splits for the lane's two columns (byte offsets vo and vo + 32 in rs, splits sb
// bytes apart from split q0 on), the loads all issued before the adds; splits from `valid` on are
// loaded clamped and not added. POL LD_SC1: the loads read the memory side, where the other
// workgroups' write-through stores went; buffer loads take the split offsets in scalar registers,
// so no vector instruction computes an address.

template <bool FULL, int POL>
__device__ __forceinline__ void lin_sum16(__amdgpu_buffer_rsrc_t rs, uint32_t vo, uint32_t sb, int q0, int valid,
                                          float& v0, float& v1)
{
    float t0[16], t1[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t so = sb * (uint32_t)(q0 + (FULL ? i : min(i, valid - 1)));
        t0[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vo, so, POL));
        t1[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vo + 32, so, POL));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (FULL || i < valid) {
            v0 += t0[i];
            v1 += t1[i];
        }
}

// Output epilogue of row m of a column group: the row's k-split partials summed in split order
// (one memory round trip per 16 splits), C to fp16, Hadamard, fp16 svh product. POL: LD_SC1 in
// the launch that wrote the partials (run by the group's last workgroup after its arrival, where
// every instruction is on the call's critical path), 0 in a launch of its own.
template <int POL>
__device__ __forceinline__ void lin_epilogue_row(const LinParams& p, int cg, int m, const float (&sv)[2])
{
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rs = weight_rsrc((const uint32_t*)p.part);
    const uint32_t vo = 4u * (uint32_t)(m * p.out + cg * 128 + lane_col(lane, 0));   // column 1: + 32 bytes
    const uint32_t sb = 4u * (uint32_t)(p.rows * p.out);
    float v0 = 0.0f, v1 = 0.0f;
    for (int q0 = 0; q0 < p.ks; q0 += 16) {
        if (q0 + 16 <= p.ks) lin_sum16<true, POL>(rs, vo, sb, q0, 16, v0, v1);
        else lin_sum16<false, POL>(rs, vo, sb, q0, p.ks - q0, v0, v1);
    }
    v0 = h2f(f2h(v0));                  // C in fp16
    v1 = h2f(f2h(v1));
    had128_lane(v0, v1, lane);
    half_t* y = p.y + (size_t)m * p.out + cg * 128 + lane_col(lane, 0);
    y[0] = f2h(h2f(f2h(v0)) * sv[0]);
    y[8] = f2h(h2f(f2h(v1)) * sv[1]);
}

// After a workgroup's waves stored their partials: wait until every store is acknowledged, arrive
// at the column group's counter, and run the epilogue if last (the stores of every workgroup of
// the group then precede the loads). One row: wave 0 arrives and runs the epilogue alone, with no
// second barrier; two: the arrival is shared through LDS and wave m runs row m.
template <int TM>
__device__ __forceinline__ void lin_arrive(const LinParams& p, int cg, int n, const float (&sv)[2])
{
    unsigned long long* word = p.arrive + (size_t)cg * ARRIVE_STRIDE;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (TM == 1) {
        if (wave != 0) return;
        int l = 0;
        if (threadIdx.x == 0) l = arrive_last(word, (unsigned)n);
        if (__builtin_amdgcn_readfirstlane(l)) lin_epilogue_row<LD_SC1>(p, cg, 0, sv);
    } else {
        __shared__ int last;
        if (threadIdx.x == 0) last = arrive_last(word, (unsigned)n);
        __syncthreads();
        if (last && wave < p.rows) lin_epilogue_row<LD_SC1>(p, cg, wave, sv);
    }
}

// The lane's two svh values, loaded at the start of the launch (the epilogue needs them only in
// the last workgroup, but then without waiting for them).
__device__ __forceinline__ void lin_load_sv(const LinParams& p, int cg, float (&sv)[2])
{
    const int lane = threadIdx.x & 63;
    sv[0] = h2f(p.svh[cg * 128 + lane_col(lane, 0)]);
    sv[1] = h2f(p.svh[cg * 128 + lane_col(lane, 1)]);
}

// Decode path: one workgroup of four waves per (128 output columns, quarter q of the k-splits),
// wave w taking split 4q + w (waves past the last split only arrive); each row's reduction order
// depends only on in/out, never on how many rows share the call. One kernel per rate (the host
// picks it). TM (1 or 2) rows: inputs rotated in the wave.
template <int K2, int TM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void lin_gemv_kernel(LinParams p)
{
    __shared__ uint32_t xl[4][TM * LIN_CW * 64];
    const int nq = (p.ks + 3) >> 2;
    const int cg = blockIdx.x / nq, q = blockIdx.x % nq;
    const int ks = __builtin_amdgcn_readfirstlane(4 * q + (threadIdx.x >> 6));
    float sv[2];
    lin_load_sv(p, cg, sv);
    if (ks < p.ks) {
        const int nch = p.in / 128;
        const int c0 = nch * ks / p.ks, c1 = nch * (ks + 1) / p.ks;
        lin_item<K2, TM>(p, cg, ks, c0, c1, xl[threadIdx.x >> 6]);
    }
    lin_arrive<TM>(p, cg, nq, sv);
}

// 3 to LIN_GEMV_ROWS rows: the rows rotated beforehand (lin_rotate_kernel), read through
// scalar loads (wider row blocks in LDS would not fit the register budget); one wave per (128
// output columns, k-split), the output epilogue in a launch of its own (lin_epilogue_kernel). At
// these row counts the last workgroup of a column group would run many rows' epilogues one after
// another (16 rows at 2048 x 7168: 38.6 us per call, against 32.1 us with the epilogue launch).
template <int K2, int TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void lin_gemv_rows_kernel(LinParams p)
{
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.ks) return;
    const int cg = __builtin_amdgcn_readfirstlane(wid / p.ks), ks = __builtin_amdgcn_readfirstlane(wid % p.ks);
    const int nch = p.in / 128;
    const int c0 = nch * ks / p.ks, c1 = nch * (ks + 1) / p.ks;
    gemv_chunk<K2, TMAX>(p.trellis, p.out / 16, cg, c0, c1, GlobalRows{p.xr, (size_t)p.in, p.xsum, nch}, k_iota64,
                         p.rows, p.part + (size_t)ks * p.rows * p.out, (size_t)p.out);
}

// One wave per (row, 128 output columns).
__global__ __launch_bounds__(256) void lin_epilogue_kernel(LinParams p)
{
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.rows) return;
    const int m = wid / ncg, cg = wid % ncg;
    float sv[2];
    lin_load_sv(p, cg, sv);
    lin_epilogue_row<0>(p, cg, m, sv);
}

// Decode path launches of one rate: up to 2 rows one launch (workgroups per (column group, 4
// splits)); 3 to 16 rows the GEMV (a wave per (column group, split)) and the epilogue.
template <int K2>
void launch_gemv_rate(const LinParams& p, hipStream_t stream)
{
    const int ncg = p.out / 128;
    if (p.rows <= LIN_ROT_ROWS) {
        const dim3 grid((unsigned)(ncg * ((p.ks + 3) / 4)));
        if (p.rows == 1) hipLaunchKernelGGL((lin_gemv_kernel<K2, 1>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((lin_gemv_kernel<K2, 2>), grid, dim3(256), 0, stream, p);
        return;
    }
    const dim3 grid((unsigned)((ncg * p.ks + 3) / 4));
    if (p.rows <= 4) hipLaunchKernelGGL((lin_gemv_rows_kernel<K2, 4>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((lin_gemv_rows_kernel<K2, 8>), grid, dim3(256), 0, stream, p);
    hipLaunchKernelGGL(lin_epilogue_kernel, dim3((unsigned)((ncg * p.rows + 3) / 4)), dim3(256), 0, stream, p);
}

// ---------------------------------------------------------------------------------------------
// More than LIN_GEMV_ROWS rows (and the rotation of 3 to LIN_GEMV_ROWS rows).

constexpr int LM_WAVES = 8;           // waves (k-ranges) per workgroup of the MFMA path

// fp16(H128(fp16(x * suh))) of every (row, 128-chunk) with the chunk's sum: one wave each.
__global__ __launch_bounds__(256) void lin_rotate_kernel(LinParams p)
{
    const int lane = threadIdx.x & 63;
    const int item = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nch = p.in / 128;
    if (item >= p.rows * nch) return;
    const int r = item / nch, c = item % nch;
    const uint32_t xw = ((const uint32_t*)(p.x + (size_t)r * p.in + c * 128))[lane];
    const uint32_t sw = ((const uint32_t*)(p.suh + c * 128))[lane];
    const half2_t xx = __builtin_bit_cast(half2_t, xw), su = __builtin_bit_cast(half2_t, sw);
    float v0 = h2f(f2h(h2f(xx.x) * h2f(su.x)));        // fp16 product
    float v1 = h2f(f2h(h2f(xx.y) * h2f(su.y)));
    had128_pair(v0, v1, lane);
    const half2_t o = {f2h(v0), f2h(v1)};
    ((uint32_t*)(p.xr + (size_t)r * p.in + c * 128))[lane] = __builtin_bit_cast(uint32_t, o);
    const float sum = wave_sum(h2f(o.x) + h2f(o.y));
    if (lane == 0) p.xsum[(size_t)r * nch + c] = sum;
}

// One workgroup per (tile of up to 64 rows, 128 output columns); wave w < p.ks streams the
// 128-chunks [nch w / ks, nch (w + 1) / ks) into MFMA accumulators and forms its partials
// (codebook map with its rows' activation sums); the partials meet in LDS, added in wave order,
// and every wave then runs the output epilogue of some of the tile's rows.
template <int K2, int MB>
__device__ __forceinline__ void lin_mfma_tile(const LinParams& p, int r0, int rows, int cg, uint32_t* stage,
                                              float (*red)[132])
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m16 = lane & 15, g = lane >> 4;
    const int nch = p.in / 128;
    const GlobalRows src{p.xr + (size_t)r0 * p.in, (size_t)p.in, p.xsum + (size_t)r0 * nch, nch};
    float pv[MB][8][4];
    if (wave < p.ks) {
        const int c0 = nch * wave / p.ks, c1 = nch * (wave + 1) / p.ks;
        f32x4_t acc[MB][8];
        mfma_accumulate<K2, MB, false>(p.trellis, p.out / 16, cg, 8 * c0, 8 * c1, src, k_iota64, rows, stage, acc);
        float xs[MB][4];
        mfma_row_sums<MB>(src, k_iota64, rows, 8 * c0, 8 * (c1 - c0), xs);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) pv[mb][nb][r] = mul1_affine(acc[mb][nb][r], xs[mb][r]);
    }
    for (int w = 0; w < p.ks; ++w) {
        __syncthreads();
        if (wave == w) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * mb + 4 * g + r;
                    if (row < rows) {
#pragma unroll
                        for (int nb = 0; nb < 8; ++nb) {
                            float* d = &red[row][16 * nb + m16];
                            *d = w == 0 ? pv[mb][nb][r] : *d + pv[mb][nb][r];
                        }
                    }
                }
        }
    }
    __syncthreads();
    float sv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) sv[h] = h2f(p.svh[cg * 128 + lane_col(lane, h)]);
    for (int row = wave; row < rows; row += LM_WAVES) {
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) v[h] = h2f(f2h(red[row][lane_col(lane, h)]));     // C in fp16
        had128_lane(v[0], v[1], lane);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            p.y[(size_t)(r0 + row) * p.out + cg * 128 + lane_col(lane, h)] = f2h(h2f(f2h(v[h])) * sv[h]);
    }
}

template <int K2>
__device__ __forceinline__ void lin_mfma_rows(const LinParams& p, int r0, int rows, int cg, uint32_t* stage,
                                              float (*red)[132])
{
    switch (__builtin_amdgcn_readfirstlane((rows + 15) >> 4)) {
        case 1: lin_mfma_tile<K2, 1>(p, r0, rows, cg, stage, red); break;
        case 2: lin_mfma_tile<K2, 2>(p, r0, rows, cg, stage, red); break;
        case 3: lin_mfma_tile<K2, 3>(p, r0, rows, cg, stage, red); break;
        default: lin_mfma_tile<K2, 4>(p, r0, rows, cg, stage, red); break;
    }
}

__global__ __launch_bounds__(64 * LM_WAVES) void lin_mfma_kernel(LinParams p)
{
    __shared__ uint32_t stage[LM_WAVES][MF_LDS_WORDS];
    __shared__ float red[64][132];      // padded rows: the partial stores hit 64 distinct banks
    const int ncg = p.out / 128;
    const int tile = blockIdx.x / ncg, cg = blockIdx.x % ncg;
    const int r0 = 64 * tile, rows = p.rows - r0 < 64 ? p.rows - r0 : 64;
    uint32_t* st = stage[threadIdx.x >> 6];
    switch (p.k2) {
        case 3: lin_mfma_rows<3>(p, r0, rows, cg, st, red); break;
        case 4: lin_mfma_rows<4>(p, r0, rows, cg, st, red); break;
        case 5: lin_mfma_rows<5>(p, r0, rows, cg, st, red); break;
        case 6: lin_mfma_rows<6>(p, r0, rows, cg, st, red); break;
        case 7: lin_mfma_rows<7>(p, r0, rows, cg, st, red); break;
        case 8: lin_mfma_rows<8>(p, r0, rows, cg, st, red); break;
        case 10: lin_mfma_rows<10>(p, r0, rows, cg, st, red); break;
        default: break;                 // the rate is validated on the host
    }
}

// k-split of a call: decode path, enough splits to fill the device once; MFMA path, one k-range
// per wave of the workgroup. Both depend on in/out only.
int linear_ksplit(int rows, int in, int out)
{
    const int ncg = out / 128, nch = in / 128;
    if (rows > LIN_GEMV_ROWS) return nch < LM_WAVES ? nch : LM_WAVES;
    int ks = (4096 + ncg - 1) / ncg;
    if (ks > nch) ks = nch;
    if (ks < 1) ks = 1;
    return ks;
}

// Workspace: the column groups' arrival counters (out/128 of them, 128 bytes apart, at offset 0
// for every row count, so that no other layout overwrites them); from 3 rows the rotated rows
// [rows][in] fp16 and their 128-chunk sums [rows][in/128]; up to 16 rows the fp32 partials
// [ks][rows][out].
static size_t arrive_bytes(int out) { return (size_t)(out / 128) * ARRIVE_STRIDE * 8; }

size_t linear_workspace(int rows, int in, int out, size_t* off_part, size_t* off_sum)
{
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    size_t o = al(arrive_bytes(out));
    if (off_sum) *off_sum = 0;
    if (off_part) *off_part = 0;
    if (rows > LIN_ROT_ROWS) {
        o = al(o + (size_t)rows * in * 2);
        if (off_sum) *off_sum = o;
        o = al(o + (size_t)rows * (in / 128) * 4);
    }
    if (rows <= LIN_GEMV_ROWS) {
        if (off_part) *off_part = o;
        o = al(o + (size_t)linear_ksplit(rows, in, out) * rows * out * 4);
    }
    return o;
}

int launch_linear(const void* x, int rows, int in, int out, const void* trellis, const void* suh,
                  const void* svh, int k2, void* y, void* ws, hipStream_t stream)
{
    LinParams p;
    size_t off_part, off_sum;
    linear_workspace(rows, in, out, &off_part, &off_sum);
    p.x = (const half_t*)x;
    p.rows = rows; p.in = in; p.out = out; p.k2 = k2;
    p.ks = linear_ksplit(rows, in, out);
    p.trellis = (const uint32_t*)trellis;
    p.suh = (const half_t*)suh;
    p.svh = (const half_t*)svh;
    p.y = (half_t*)y;
    const size_t off_xr = (arrive_bytes(out) + 255) & ~(size_t)255;
    p.arrive = (unsigned long long*)ws;
    p.xr = rows > LIN_ROT_ROWS ? (half_t*)((char*)ws + off_xr) : nullptr;
    p.xsum = rows > LIN_ROT_ROWS ? (float*)((char*)ws + off_sum) : nullptr;
    p.part = rows <= LIN_GEMV_ROWS ? (float*)((char*)ws + off_part) : nullptr;
    if (rows > LIN_ROT_ROWS) {
        const long waves = (long)rows * (in / 128);
        hipLaunchKernelGGL(lin_rotate_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, p);
    }
    if (rows > LIN_GEMV_ROWS) {
        const long tiles = (rows + 63) / 64;
        hipLaunchKernelGGL(lin_mfma_kernel, dim3((unsigned)(tiles * (out / 128))), dim3(64 * LM_WAVES), 0, stream, p);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    switch (k2) {
        case 3: launch_gemv_rate<3>(p, stream); break;
        case 4: launch_gemv_rate<4>(p, stream); break;
        case 5: launch_gemv_rate<5>(p, stream); break;
        case 6: launch_gemv_rate<6>(p, stream); break;
        case 7: launch_gemv_rate<7>(p, stream); break;
        case 8: launch_gemv_rate<8>(p, stream); break;
        case 10: launch_gemv_rate<10>(p, stream); break;
        default: return -1;             // the rate is validated by the caller
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
