/*
 * Scalar C restatement of the EXL3 trellis decode (TEST INFRASTRUCTURE ONLY).
 *
 * Independent of the numpy oracle (oracle/exl3.py): the codebook rounds to fp16 with a
 * hand-written round-to-nearest-even, and windows are extracted two ways, per position
 * (the scalar `dq`, exl3_dq.cuh:15-31) and in groups of eight from one or two funnel shifts
 * followed by shift chains (the 8-wide forms, exl3_dq.cuh:96-285). Tests require all of
 * them to agree with the numpy extractors bit for bit.
 *
 * Reference files: runtime/ds41/csrc/moe_coop3072/vendor/quant/{codebook,exl3_dq}.cuh.
 * Build: oracle/Makefile (gcc only; output in oracle/_build/).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

/* fp32 -> fp16 bits, round to nearest even (normal, subnormal, overflow to inf). */
static uint16_t f32_to_f16_bits(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) x = sign;
        else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) x = sign | 0x7f800000u | (man << 13);
    else x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* MUL1 codebook, codebook.cuh:86-99: fp16 bits of hfma(1024 + bytesum, 0x1eee, 0xc931). */
uint16_t evo_mul1_decode(uint32_t state)
{
    uint32_t p = (state & 0xffffu) * 0x83DCD12Du;
    uint32_t bs = (p & 0xff) + ((p >> 8) & 0xff) + ((p >> 16) & 0xff) + (p >> 24);
    float h = f16_bits_to_f32((uint16_t)(0x6400u + bs));
    float k = f16_bits_to_f32(0x1eee);
    float b = f16_bits_to_f32(0xc931);
    /* h*k and h*k + b are exact in fp32 (multiples of 2^-18 below 16): one fp16 rounding. */
    volatile float prod = h * k;
    volatile float sum = prod + b;
    return f32_to_f16_bits(sum);
}

void evo_codebook(uint16_t* out65536)
{
    for (uint32_t s = 0; s < 65536u; ++s) out65536[s] = evo_mul1_decode(s);
}

static int tile_words_k2(int k2)          /* k2 = 2K */
{
    return (k2 & 1) ? 4 * k2 : 4 * k2;    /* 8K for integer K, 4(2b+1) for b+0.5: both 4*k2 */
}

static int64_t end_bit(int k2, int p)
{
    if (!(k2 & 1)) return (int64_t)(p + 1) * (k2 / 2);
    int b = k2 / 2, b2 = 2 * b + 1;
    return (p & 1) ? (int64_t)((p + 1) / 2) * b2 : (int64_t)(p / 2) * b2 + b;
}

static uint32_t funnel(uint32_t hi, uint32_t lo, int s)
{
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> s);
}

/* Per-position window (exl3_dq.cuh:15-31, generalised to half rates by the end bit). */
uint16_t evo_state_scalar(const uint32_t* tile, int k2, int p)
{
    int tw = tile_words_k2(k2);
    int64_t nbits = 32 * (int64_t)tw;
    int64_t e = end_bit(k2, p) + nbits;
    int64_t b0 = e - 16, b1 = e;
    int i0 = (int)((b0 / 32) % tw);
    int i1 = (int)(((b1 - 1) / 32) % tw);
    int s = (int)(((b1 - 1) / 32 + 1) * 32 - b1);
    return (uint16_t)(funnel(tile[i0], tile[i1], s) & 0xffffu);
}

/*
 * Eight windows of positions t_offset .. t_offset+7 (t_offset a multiple of 8) from at most
 * two word pairs: the last window by a funnel shift, the others by right shifts of that
 * value (exl3_dq.cuh:96-161 integer K; 254-285 rate b+0.5). Each half of the group (four
 * windows, 16 + 3K bits, plus up to 31 bits of alignment) is read from one 64-bit word pair,
 * as the reference's dq4 does (exl3_dq.cuh:52-72); that fits for K <= 5, and wider integer
 * rates return -1.
 */
int evo_states_group8(const uint32_t* tile, int k2, int t_offset, uint16_t* out8)
{
    int tw = tile_words_k2(k2);
    int64_t nbits = 32 * (int64_t)tw;
    if (k2 & 1) {
        int ka = k2 / 2, b2 = 2 * ka + 1, gspan = 18 + 3 * ka;
        int64_t e7 = (int64_t)((t_offset >> 1) + 4) * b2 + 128 * b2;
        int64_t e3 = e7 - 2 * b2;
        int64_t ends[2] = {e3, e7};
        for (int g = 0; g < 2; ++g) {
            int64_t e = ends[g];
            int hi = (int)(((e - 1) / 32) % tw), lo = (int)(((e - gspan) / 32) % tw);
            int s = (int)(((e - 1) / 32 + 1) * 32 - e);
            uint32_t w3 = funnel(tile[lo], tile[hi], s);
            uint32_t w2 = w3 >> (ka + 1);
            uint32_t w1 = w2 >> ka;
            uint32_t w0 = w1 >> (ka + 1);
            out8[4 * g + 0] = (uint16_t)(w0 & 0xffff);
            out8[4 * g + 1] = (uint16_t)(w1 & 0xffff);
            out8[4 * g + 2] = (uint16_t)(w2 & 0xffff);
            out8[4 * g + 3] = (uint16_t)(w3 & 0xffff);
        }
        return 0;
    }
    int K = k2 / 2;
    if (K > 5) return -1;          /* 16 + 3K + 31 > 64: the two-word group form needs K <= 5 */
    for (int g = 0; g < 2; ++g) {
        int64_t e = (int64_t)(t_offset + 4 * g + 4) * K + nbits;   /* end of the group's last window */
        int64_t first = e - 16 - 3 * K;
        int hi = (int)((first / 32) % tw), lo = (int)(((e - 1) / 32) % tw);
        int s = (int)(((e - 1) / 32 + 1) * 32 - e);
        uint32_t w3 = funnel(tile[hi], tile[lo], s);
        out8[4 * g + 3] = (uint16_t)(w3 & 0xffff);
        out8[4 * g + 2] = (uint16_t)((w3 >> K) & 0xffff);
        out8[4 * g + 1] = (uint16_t)((w3 >> (2 * K)) & 0xffff);
        out8[4 * g + 0] = (uint16_t)((w3 >> (3 * K)) & 0xffff);
    }
    return 0;
}

/* Tile position -> (k, n) (fragment layout; see oracle/exl3.py tile_coords). */
static void coords(int p, int* k, int* n)
{
    int lane = p >> 3, j = p & 7, g = lane >> 2, t = lane & 3;
    *k = 2 * t + (j & 1) + 8 * ((j >> 1) & 1);
    *n = g + 8 * (j >> 2);
}

/* Dequantize trellis int16 [in/16][out/16][16*K or 16b+8] -> fp16 bits W[in][out]. */
int evo_dequant(const int16_t* trellis, int in, int out, int k2, uint16_t* w)
{
    if (in % 16 || out % 16 || k2 < 2 || k2 > 16) return -1;
    int tw = tile_words_k2(k2);
    int kt_n = in / 16, nt_n = out / 16;
#pragma omp parallel for schedule(static)
    for (int kt = 0; kt < kt_n; ++kt)
        for (int nt = 0; nt < nt_n; ++nt) {
            uint32_t words[64];
            const uint16_t* t16 = (const uint16_t*)trellis + ((size_t)kt * nt_n + nt) * (size_t)(2 * tw);
            for (int i = 0; i < tw; ++i) words[i] = (uint32_t)t16[2 * i] | ((uint32_t)t16[2 * i + 1] << 16);
            for (int p = 0; p < 256; ++p) {
                int k, n;
                coords(p, &k, &n);
                w[(size_t)(16 * kt + k) * out + 16 * nt + n] = evo_mul1_decode(evo_state_scalar(words, k2, p));
            }
        }
    return 0;
}

/* 128-point Hadamard, radix-2 on element bits 0..6 (lower a+b, upper a-b), scale last. */
void evo_had128(const float* in, float* out, int chunks)
{
    const float r = 0.088388347648f;
    for (int c = 0; c < chunks; ++c) {
        float v[128];
        memcpy(v, in + 128 * c, sizeof v);
        for (int h = 1; h < 128; h <<= 1)
            for (int i = 0; i < 128; ++i)
                if (!(i & h)) {
                    volatile float a = v[i], b = v[i + h];
                    v[i] = a + b;
                    v[i + h] = a - b;
                }
        for (int i = 0; i < 128; ++i) out[128 * c + i] = v[i] * r;
    }
}
