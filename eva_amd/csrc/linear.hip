// Single EXL3 linear, fp16 in / fp16 out (the config-1 layer).
//
// Reference: ELinear.forward -> LinearEXL3 (runtime/ds41/exl3_linear.py:97-131), kernel
// exl3_gemv_kernel.cuh:217-234 (input: fp16 x*suh, Hadamard, fp16), 295-459 (GEMV, fp16 C),
// 463-490 with hadamard_inner.cuh:93-147 (output Hadamard to fp16, fp16 product with svh).
// Up to 16 rows, two launches: a k-split decode GEMV whose waves rotate their own input chunks
// (fp16(H128(fp16(x * suh)))) into LDS while their first weight loads are in flight, writing
// fp32 partials; and the output epilogue (the partials summed in fixed order, fp16 C,
// Hadamard, fp16 svh product).
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
        gemv_wave<K2, TM>(p.trellis, p.out / 16, cg, 8 * w0, 8 * w1, src, tm, acc, stage);
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
            dst[col0] = mul1_affine(acc[m][0], xs[m]);
            dst[col1] = mul1_affine(acc[m][1], xs[m]);
        }
    }
}

template <int K2, int TM>
__device__ __forceinline__ void lin_item(const LinParams& p, int cg, int ks, int c0, int c1, uint32_t* lds)
{
    if constexpr (TM == 1) lin_rows<K2, 1>(p, 0, 1, cg, ks, c0, c1, lds);
    else lin_rows<K2, 2>(p, 0, p.rows, cg, ks, c0, c1, lds);
}

// One wave per (128 output columns, k-split); each row's reduction order depends only on
// in/out, never on how many rows share the call. TM (1 or 2) rows: inputs rotated in the wave.
template <int TM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void lin_gemv_kernel(LinParams p)
{
    __shared__ uint32_t xl[4][TM * LIN_CW * 64];
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.ks) return;
    const int cg = __builtin_amdgcn_readfirstlane(wid / p.ks), ks = __builtin_amdgcn_readfirstlane(wid % p.ks);
    const int nch = p.in / 128;
    const int c0 = nch * ks / p.ks, c1 = nch * (ks + 1) / p.ks;
    uint32_t* lds = xl[threadIdx.x >> 6];
    switch (p.k2) {
        case 3: lin_item<3, TM>(p, cg, ks, c0, c1, lds); break;
        case 4: lin_item<4, TM>(p, cg, ks, c0, c1, lds); break;
        case 5: lin_item<5, TM>(p, cg, ks, c0, c1, lds); break;
        case 6: lin_item<6, TM>(p, cg, ks, c0, c1, lds); break;
        case 7: lin_item<7, TM>(p, cg, ks, c0, c1, lds); break;
        case 8: lin_item<8, TM>(p, cg, ks, c0, c1, lds); break;
        case 10: lin_item<10, TM>(p, cg, ks, c0, c1, lds); break;
        default: break;                 // the rate is validated on the host
    }
}

// 3 to LIN_GEMV_ROWS rows: the rows rotated beforehand (lin_rotate_kernel), read through
// scalar loads (wider row blocks in LDS would not fit the register budget).
template <int TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void lin_gemv_rows_kernel(LinParams p)
{
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.ks) return;
    const int cg = __builtin_amdgcn_readfirstlane(wid / p.ks), ks = __builtin_amdgcn_readfirstlane(wid % p.ks);
    const int nch = p.in / 128;
    const int c0 = nch * ks / p.ks, c1 = nch * (ks + 1) / p.ks;
    gemv_dispatch_k<TMAX>(p.k2, p.trellis, p.out / 16, cg, c0, c1, GlobalRows{p.xr, (size_t)p.in, p.xsum, nch},
                          k_iota64, p.rows, p.part + (size_t)ks * p.rows * p.out, (size_t)p.out);
}

__global__ __launch_bounds__(256) void lin_epilogue_kernel(LinParams p)
{
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int ncg = p.out / 128;
    if (wid >= ncg * p.rows) return;
    const int m = wid / ncg, cg = wid % ncg;
    float sv[2];                                       // loaded with the partials
#pragma unroll
    for (int h = 0; h < 2; ++h) sv[h] = h2f(p.svh[cg * 128 + lane_col(lane, h)]);
    // the k-split partials in fixed order; the loads of up to 16 splits of both columns are issued
    // before their adds (one memory round trip per 16 splits: the call is latency-bound)
    float v[2] = {0.0f, 0.0f};
    const size_t stride = (size_t)p.rows * p.out;
    const float* pp[2] = {p.part + (size_t)m * p.out + cg * 128 + lane_col(lane, 0),
                          p.part + (size_t)m * p.out + cg * 128 + lane_col(lane, 1)};
    for (int q0 = 0; q0 < p.ks; q0 += 16) {
        float t[2][16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (q0 + i < p.ks)
#pragma unroll
                for (int h = 0; h < 2; ++h) t[h][i] = gptr<float>(pp[h])[(q0 + i) * stride];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (q0 + i < p.ks)
#pragma unroll
                for (int h = 0; h < 2; ++h) v[h] += t[h][i];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) v[h] = h2f(f2h(v[h]));    // C in fp16
    had128_lane(v[0], v[1], lane);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = cg * 128 + lane_col(lane, h);
        p.y[(size_t)m * p.out + col] = f2h(h2f(f2h(v[h])) * sv[h]);
    }
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

// Workspace: up to 2 rows, the fp32 partials [ks][rows][out]; 3 to 16 rows, also the rotated
// rows [rows][in] fp16 and their 128-chunk sums [rows][in/128]; MFMA path, those two only.
size_t linear_workspace(int rows, int in, int out, size_t* off_part, size_t* off_sum)
{
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    size_t o = 0;
    if (off_sum) *off_sum = 0;
    if (off_part) *off_part = 0;
    if (rows > LIN_ROT_ROWS) {
        o = al((size_t)rows * in * 2);
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
    p.xr = rows > LIN_ROT_ROWS ? (half_t*)ws : nullptr;
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
    {
        const int waves = (out / 128) * p.ks;
        const dim3 grid((waves + 3) / 4);
        if (rows == 1) hipLaunchKernelGGL(lin_gemv_kernel<1>, grid, dim3(256), 0, stream, p);
        else if (rows == 2) hipLaunchKernelGGL(lin_gemv_kernel<2>, grid, dim3(256), 0, stream, p);
        else if (rows <= 4) hipLaunchKernelGGL(lin_gemv_rows_kernel<4>, grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL(lin_gemv_rows_kernel<8>, grid, dim3(256), 0, stream, p);
    }
    {
        const int waves = (out / 128) * rows;
        hipLaunchKernelGGL(lin_epilogue_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace evamx
