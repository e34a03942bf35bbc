// The MFMA core shared by the prefill-shaped expert GEMMs and the large-row EXL3 linear:
// trellis decode into LDS feeding fp16 MFMA on gfx950.
//
//   - a wave streams its 8 trellis tiles per k-slice exactly like the decode GEMV (lane 8*i + q
//     owns tile i's columns q, q + 8) and decodes two k-slices into the (1024 + bytesum) fp16
//     values of the affine codebook map (w = 0x1eee * h + 0xc931);
//   - it restages them through a wave-private 8 KiB LDS region into the B operands of
//     v_mfma_f32_16x16x32_f16 (lane n + 16 g holds column n, k = 8g .. 8g+7), one per 16-column
//     tile, and reads the rotated activations of its rows as the A operands (lane m + 16 g
//     holds row m, the same k) straight from global memory;
//   - MB x 8 accumulators (16 MB rows x 128 columns, fp32) take sum_k x_k h_k; the caller
//     applies the codebook map per column with the rows' activation sums.
//
// The LDS exchange stays within a wave (a wave's LDS instructions execute in order), so the
// waves of a workgroup never synchronise inside it.
#pragma once
#include "evamx_gemv.hpp"

namespace evamx {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int MF_LDS_WORDS = 8 * 64 * 4;        // per wave: 8 B operands x 64 lanes x 16 bytes
constexpr int MF_PF = 4;                        // k-slices of weight prefetch (two MFMA k-steps)

// Accumulators of one work item: rows [0, rows) (slots slot_of[0..rows)) of activations src
// (fp16 [slot][K] with 128-chunk sums) times the (1024 + bytesum) values of tiles 8*cg .. 8*cg+7
// of a projection over the k-slices [kt0, kt1) (whole 128-chunks): acc[mb][nb][r] = sum_k x_k h_k
// for row 16 mb + 4 g + r and column 16 nb + m16 (lane = m16 + 16 g). lds: the wave's
// MF_LDS_WORDS words.
template <int K2, int MB, bool PRIO>
__device__ __forceinline__ void mfma_accumulate(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                                const GlobalRows& src, const int* __restrict__ slot_of, int rows,
                                                uint32_t* lds, f32x4_t (&acc)[MB][8])
{
    using R = Rate<K2>;
    constexpr int K = R::K;
    constexpr int TW = R::TW;
    const int lane = threadIdx.x & 63;
    const int q = lane & 7, ti = lane >> 3;       // decode layout: run q of tile ti
    const int m16 = lane & 15, g = lane >> 4;     // MFMA layout: row/column m16, k group g
    kt0 = __builtin_amdgcn_readfirstlane(kt0);
    const int nk = __builtin_amdgcn_readfirstlane(kt1) - kt0;
    const uint32_t slice = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(nt_n * TW));
    const uint32_t cbase = __builtin_amdgcn_readfirstlane(4u * (uint32_t)(cg * 8 * TW) + (uint32_t)kt0 * 4u * (uint32_t)(nt_n * TW));
    const __amdgpu_buffer_rsrc_t rsrc = weight_rsrc(trellis);
    uint32_t lane_off, prev_off, sh;
    lane_offsets<K2>(lane, lane_off, prev_off, sh);

    // A rows of this lane: m16 + 16 mb (rows past the tile read row 0; their results are dropped)
    const __attribute__((address_space(1))) u32x4_t* arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = m16 + 16 * mb;
        const int s = slot_of[r < rows ? r : 0];
        arow[mb] = (const __attribute__((address_space(1))) u32x4_t*)(src.A + (size_t)s * src.stride + 16 * kt0) + g;
    }

#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    LaneWords<K> ring[MF_PF];
    const int last = nk - 1;
#pragma unroll
    for (int d = 0; d < MF_PF; ++d)
        load_slice<K>(ring[d], rsrc, cbase + (uint32_t)min(d, last) * slice, lane_off, prev_off);

    u32x4_t a_cur[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a_cur[mb] = arow[mb][0];

    // LDS slots: B operand nb = tile ti, lane n + 16 g <- (column n = 8c + q, k group g = 2s + kh)
    uint32_t* wdst = lds + 4 * (64 * ti + q);
    const uint32_t* rsrc_lds = lds + 4 * lane;

    auto kstep = [&](int kk, LaneWords<K>& w0, LaneWords<K>& w1) {
        // next step's A operands first: their latency hides behind this step's decode
        u32x4_t a_nxt[MB];
        const int kn = kk + 1 < (nk >> 1) ? kk + 1 : kk;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a_nxt[mb] = arow[mb][4 * kn];
        wave_lds_fence();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            LaneWords<K>& w = s == 0 ? w0 : w1;
            half2_t wp[16];
            decode_slice<K2>(w, sh, wp);
            load_slice<K>(w, rsrc, cbase + (uint32_t)min(2 * kk + s + MF_PF, last) * slice, lane_off, prev_off);
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh) {
                    const u32x4_t v = {__builtin_bit_cast(uint32_t, wp[kh + 2 * c]),
                                       __builtin_bit_cast(uint32_t, wp[kh + 2 * c + 4]),
                                       __builtin_bit_cast(uint32_t, wp[kh + 2 * c + 8]),
                                       __builtin_bit_cast(uint32_t, wp[kh + 2 * c + 12])};
                    *(u32x4_t*)(wdst + 4 * (8 * c + 16 * (2 * s + kh))) = v;
                }
        }
        wave_lds_fence();
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const u32x4_t bv = *(const u32x4_t*)(rsrc_lds + 256 * nb);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a_cur[mb]),
                                                                     __builtin_bit_cast(half8_t, bv), acc[mb][nb], 0, 0, 0);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a_cur[mb] = a_nxt[mb];
    };

    // nk is a multiple of 8 (whole 128-chunks): pairs of ring slots per step, two steps per round
    for (int kk = 0; kk < (nk >> 1); kk += 2) {
        if constexpr (PRIO) progress_priority(kk, nk >> 1);
        kstep(kk, ring[0], ring[1]);
        kstep(kk + 1, ring[2], ring[3]);
    }
    if constexpr (PRIO) progress_priority(1, 1);

}

// Activation sums over the k-slices [kt0, kt0 + nk) of the rows whose accumulators a lane holds:
// xs[mb][r] for row 16 mb + 4 g + r (lane = m16 + 16 g). Lane (m16, g) first sums chunks c0 + g,
// c0 + g + 4, ... of row m16 + 16 mb; the four k groups are summed across lanes; then each
// lane fetches the sums of its output rows.
template <int MB>
__device__ __forceinline__ void mfma_row_sums(const GlobalRows& src, const int* __restrict__ slot_of, int rows, int kt0,
                                              int nk, float (&xs)[MB][4])
{
    const int lane = threadIdx.x & 63;
    const int m16 = lane & 15, g = lane >> 4;
    const int c0 = kt0 >> 3, c1 = c0 + (nk >> 3);
    float v[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = m16 + 16 * mb;
        const int s = slot_of[r < rows ? r : 0];
        float t = strided_sum<8>(src.sums + (size_t)s * src.sums_stride, c0 + g, c1, 4);
        t = pair_sum<16>(t, lane);
        t = pair_sum<32>(t, lane);
        v[mb] = t;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) xs[mb][r] = __shfl(v[mb], 4 * g + r, WAVE);
}

// One work item with its partials stored: part[slot * part_stride + 128 * cg + column] =
// 0x1eee * acc + 0xc931 * (row's activation sum), for rows < rows.
template <int K2, int MB, bool PRIO>
__device__ __forceinline__ void mfma_item(const uint32_t* __restrict__ trellis, int nt_n, int cg, int kt0, int kt1,
                                          const GlobalRows& src, const int* __restrict__ slot_of, int rows,
                                          float* __restrict__ part, size_t part_stride, uint32_t* lds)
{
    f32x4_t acc[MB][8];
    mfma_accumulate<K2, MB, PRIO>(trellis, nt_n, cg, kt0, kt1, src, slot_of, rows, lds, acc);
    kt0 = __builtin_amdgcn_readfirstlane(kt0);
    const int nk = __builtin_amdgcn_readfirstlane(kt1) - kt0;
    float xs[MB][4];
    mfma_row_sums<MB>(src, slot_of, rows, kt0, nk, xs);
    const int lane = threadIdx.x & 63;
    const int m16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * mb + 4 * g + r;
            if (row < rows) {
                float* dst = part + (size_t)slot_of[row] * part_stride + 128 * cg + m16;
#pragma unroll
                for (int nb = 0; nb < 8; ++nb) dst[16 * nb] = mul1_affine(acc[mb][nb][r], xs[mb][r]);
            }
        }
    }
}

}  // namespace evamx
