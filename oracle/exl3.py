"""EXL3 trellis format and MUL1 codebook: CPU restatement (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): this module is the
checker for the HIP kernels, never part of the product path.

Each function cites the reference file:line it restates. Abbreviations:

- ``codebook.cuh``      = runtime/ds41/csrc/moe_coop3072/vendor/quant/codebook.cuh
- ``exl3_dq.cuh``       = runtime/ds41/csrc/moe_coop3072/vendor/quant/exl3_dq.cuh
- ``K.cuh``             = runtime/ds41/csrc/moe_coop3072/vendor/quant/exl3_moe_coop_kernel.cuh
- ``hadamard_inner.cuh``= runtime/ds41/csrc/moe_coop3072/vendor/quant/hadamard_inner.cuh
- ``ptx_rocm.cuh``      = runtime/ds41/csrc/moe_coop3072/vendor/rocm/ptx_rocm.cuh

Pinning (tests/test_oracle_exl3.py):

- codebook: exhaustive over all 65 536 states against the reference's integer
  identity ``mul1_integer`` (cpu_precision_reference.py:43-45) within its
  published 0.0028 gap, plus exact closed-form invariants, plus the scalar C
  restatement (``exl3_oracle.c``) bit for bit;
- bit windows: two independent extractors (``tile_states_funnel`` - per
  position funnel shift; ``tile_states_bits`` - explicit MSB-first bit string)
  agree on every position of random tiles of every K, and the C scalar and
  8-wide group forms agree with both;
- tile map: bijection onto the 16x16 tile, and the fragment-layout derivation;
- Hadamard: equals the Sylvester matrix (scipy.linalg.hadamard) to fp32
  rounding and is its own inverse.
"""
from __future__ import annotations

import numpy as np

MUL1_MULT = 0x83DCD12D          # codebook.cuh:88
MUL1_ACC = 0x6400               # codebook.cuh:89 (fp16 1024.0)
K_INV_BITS = 0x1EEE             # codebook.cuh:95 (fp16 0.00676727...)
K_BIAS_BITS = 0xC931            # codebook.cuh:96 (fp16 -10.3828125)
R_SCALE = np.float32(0.088388347648)   # K.cuh:48, 1/sqrt(128) as the reference spells it

HALF_RATES = (1.5, 2.5, 3.5)
INT_RATES = (1, 2, 3, 4, 5, 6, 7, 8)


def fp16_from_bits(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


K_INV = float(fp16_from_bits(K_INV_BITS))
K_BIAS = float(fp16_from_bits(K_BIAS_BITS))


# ----------------------------------------------------------------------------------------------
# Codebook


def mul1_bytesum(states) -> np.ndarray:
    """Byte sum of ``state * 0x83DCD12D mod 2^32`` (codebook.cuh:88-94, dp4a with 0x01010101)."""
    s = np.asarray(states, dtype=np.uint64) & np.uint64(0xFFFF)
    p = (s * np.uint64(MUL1_MULT)) & np.uint64(0xFFFFFFFF)
    return ((p & np.uint64(0xFF)) + ((p >> np.uint64(8)) & np.uint64(0xFF))
            + ((p >> np.uint64(16)) & np.uint64(0xFF)) + (p >> np.uint64(24))).astype(np.int64)


def mul1_decode(states) -> np.ndarray:
    """fp16 weight of each 16-bit trellis state (codebook.cuh:86-99).

    ``h = fp16_bits(0x6400 + bytesum)`` is exactly ``1024 + bytesum``; the weight is
    ``__hfma(h, 0x1eee, 0xc931)``: one fp16 rounding of ``h*k + b``. The product and sum
    are exact in float64 (both are multiples of 2^-18 below 2^11), so a single
    float64 -> float16 round-to-nearest-even reproduces the fused fp16 FMA.
    """
    h = 1024.0 + mul1_bytesum(states).astype(np.float64)
    return (h * K_INV + K_BIAS).astype(np.float16)


_LUT = None


def codebook_lut() -> np.ndarray:
    """All 65 536 decoded weights, indexed by state (read-only array)."""
    global _LUT
    if _LUT is None:
        _LUT = mul1_decode(np.arange(65536, dtype=np.uint32))
        _LUT.setflags(write=False)
    return _LUT


# ----------------------------------------------------------------------------------------------
# Bit-rate geometry


def check_rate(K: float) -> float:
    K = float(K)
    if K in INT_RATES or K in HALF_RATES:
        return K
    raise ValueError(f"unsupported EXL3 bit rate {K}")


def is_half(K: float) -> bool:
    return float(K) in HALF_RATES


def tile_words(K: float) -> int:
    """uint32 words per 16x16 tile (K.cuh:360): 8K, or 4(2b+1) at rate b+0.5."""
    K = check_rate(K)
    return 4 * (2 * int(K) + 1) if is_half(K) else 8 * int(K)


def tile_u16(K: float) -> int:
    """int16 entries per tile in the ``trellis [in/16, out/16, T]`` layout (model.py:973-983)."""
    return 2 * tile_words(K)


def position_end_bits(K: float) -> np.ndarray:
    """Exclusive end bit of each position's 16-bit window inside the tile's bit string.

    Integer rate: ``(p+1)K`` (exl3_dq.cuh:18-19). Rate b+0.5: positions alternate b and b+1
    bits with the odd positions carrying the extra bit (exl3_dq.cuh:254-275), so an odd
    position 2q+1 ends at ``(q+1)(2b+1)`` and an even position 2q at ``q(2b+1)+b``.
    """
    K = check_rate(K)
    p = np.arange(256, dtype=np.int64)
    if not is_half(K):
        return (p + 1) * int(K)
    b = int(K)
    b2 = 2 * b + 1
    return np.where(p % 2 == 1, (p + 1) // 2 * b2, (p // 2) * b2 + b)


def window_plan(K: float):
    """Per position: (word holding the first window bit, word holding the last, right shift).

    The tile is a circular bit string of 32*TW bits; global bit g is bit ``31 - g%32`` of
    word ``g//32`` (MSB first: the funnel shifts of exl3_dq.cuh:5-13,25-29). The state is the
    16 bits ending at the position's end bit; windows of the first positions wrap to the
    tile's tail (exl3_dq.cuh:18,25-26: ``+ 256*bits`` and ``% (bits*256/32)``).
    """
    tw = tile_words(K)
    nbits = 32 * tw
    end = position_end_bits(K) + nbits          # keep positive before the modulo
    first = end - 16
    last = end - 1
    i_hi = (first // 32) % tw
    i_lo = (last // 32) % tw
    shift = 32 * (last // 32 + 1) - end
    return i_hi.astype(np.int64), i_lo.astype(np.int64), shift.astype(np.int64)


def tile_states_funnel(words, K: float) -> np.ndarray:
    """States of all 256 positions of each tile: ``words [..., TW] uint32 -> [..., 256] uint16``.

    Funnel-shift form of ``dq`` (exl3_dq.cuh:15-31): ``((hi << 32 | lo) >> s) & 0xffff``.
    """
    w = np.asarray(words, dtype=np.uint32)
    if w.shape[-1] != tile_words(K):
        raise ValueError("last axis must be the tile's words")
    i_hi, i_lo, s = window_plan(K)
    hi = w[..., i_hi].astype(np.uint64)
    lo = w[..., i_lo].astype(np.uint64)
    return (((hi << np.uint64(32)) | lo) >> s.astype(np.uint64) & np.uint64(0xFFFF)).astype(np.uint16)


def tile_states_bits(words, K: float) -> np.ndarray:
    """Independent extractor over an explicit bit string (same contract as the funnel form)."""
    w = np.asarray(words, dtype=np.uint32)
    tw = tile_words(K)
    if w.shape[-1] != tw:
        raise ValueError("last axis must be the tile's words")
    lead = w.shape[:-1]
    be = w.reshape(-1, tw).astype(">u4").view(np.uint8).reshape(-1, tw * 4)
    bits = np.unpackbits(be, axis=1)                       # MSB-first per byte == per word
    nbits = 32 * tw
    end = position_end_bits(K)
    idx = (end[:, None] - 16 + np.arange(16)[None, :]) % nbits   # [256, 16], oldest bit first
    sel = bits[:, idx].astype(np.uint32)                   # [n, 256, 16]
    weights = (1 << np.arange(15, -1, -1)).astype(np.uint32)
    states = (sel * weights).sum(axis=2).astype(np.uint16)
    return states.reshape(*lead, 256)


# ----------------------------------------------------------------------------------------------
# Tile position -> matrix coordinate


def tile_coords():
    """(k, n) inside the 16x16 tile of every position p.

    ``lane = p >> 3`` owns positions 8*lane..8*lane+7 (``t_offset = lane << 3``, K.cuh:472);
    they decode in order into fragments f0 = (d0d1, d2d3), f1 = (d4d5, d6d7)
    (exl3_dq.cuh:153-160). With g = lane/4, t = lane%4 the B fragment element
    ``b[i] = {B[2t+8i][g], B[2t+8i+1][g]}`` (ptx_rocm.cuh:13); f0 multiplies columns 0..7 and
    f1 columns 8..15 (K.cuh:494-495,513-514). Hence k = 2t + (j&1) + 8((j>>1)&1) and
    n = g + 8(j>>2), j = p & 7.
    """
    p = np.arange(256)
    lane, j = p >> 3, p & 7
    g, t = lane >> 2, lane & 3
    k = 2 * t + (j & 1) + 8 * ((j >> 1) & 1)
    n = g + 8 * (j >> 2)
    return k.astype(np.int64), n.astype(np.int64)


def trellis_words(trellis) -> np.ndarray:
    """View int16 ``[in/16, out/16, T]`` as uint32 words: ``u16[2w] | u16[2w+1] << 16`` (K.cuh:751)."""
    t = np.ascontiguousarray(np.asarray(trellis))
    if t.dtype not in (np.int16, np.uint16):
        raise TypeError("trellis must be int16/uint16")
    u = t.view(np.uint16).astype(np.uint32)
    return u[..., 0::2] | (u[..., 1::2] << np.uint32(16))


def trellis_states(trellis, K: float) -> np.ndarray:
    """States ``[in/16, out/16, 256]`` of a whole projection."""
    return tile_states_funnel(trellis_words(trellis), K)


def dequant(trellis, K: float) -> np.ndarray:
    """Decoded fp16 weight ``W[k][n]`` of shape ``[in, out]`` (the bit-exact dequant contract).

    The tile at (kt, nt) sits at word offset ``(kt*(out/16) + nt)*TW`` (K.cuh:377,404).
    """
    t = np.asarray(trellis)
    kt, nt, t16 = t.shape
    if t16 != tile_u16(K):
        raise ValueError(f"trellis last dim {t16} does not match K={K}")
    vals = codebook_lut()[trellis_states(t, K)]            # [kt, nt, 256]
    kk, nn = tile_coords()
    tiles = np.empty((kt, nt, 16, 16), dtype=np.float16)
    tiles[:, :, kk, nn] = vals
    return tiles.transpose(0, 2, 1, 3).reshape(kt * 16, nt * 16)


def pack_tile_bitstring(bits) -> np.ndarray:
    """Pack an MSB-first bit string of 32*TW bits into uint32 words (inverse of the bit view)."""
    b = np.asarray(bits, dtype=np.uint8).reshape(-1, 32)
    weights = (1 << np.arange(31, -1, -1, dtype=np.uint64))
    return (b.astype(np.uint64) * weights).sum(axis=1).astype(np.uint32)


# ----------------------------------------------------------------------------------------------
# Hadamard


def had128(v) -> np.ndarray:
    """Sylvester H128 over each 128-chunk of the last axis, reference fp32 evaluation order.

    Element e = 4*lane + i. Stage on bit 0 and bit 1 locally (s0=v0+v1, d0=v0-v1, ...;
    K.cuh:134-141), then lane bits 0..4 (e bits 2..6) by xor butterflies where the lower
    index keeps ``a + b`` and the upper gets ``(-own) + partner = a - b``
    (hadamard_inner.cuh:17-44), and the scale last (K.cuh:143-146). Equivalently: radix-2
    butterflies on e bits 0, 1, ..., 6 in that order, all in fp32.
    """
    x = np.asarray(v, dtype=np.float32)
    if x.shape[-1] % 128:
        raise ValueError("last axis must be a multiple of 128")
    lead = x.shape[:-1]
    y = x.reshape(-1, 128).copy()
    h = 1
    while h < 128:
        z = y.reshape(-1, 128 // (2 * h), 2, h)
        a = z[:, :, 0, :].copy()
        b = z[:, :, 1, :].copy()
        z[:, :, 0, :] = a + b
        z[:, :, 1, :] = a - b
        y = z.reshape(-1, 128)
        h *= 2
    y = y * R_SCALE
    return y.reshape(*lead, x.shape[-1]).astype(np.float32)


def round_fp16(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float32).astype(np.float16)
