"""Pins the EXL3 oracle (``oracle/exl3.py``, ``oracle/exl3_oracle.c``) without trusting it.

The reference ships no golden vectors for this path (its tests omit the MoE kernels), so
each oracle function is checked against something that fixes it independently:

- codebook: the reference's own integer identity ``mul1_integer``
  (runtime/ds41/cpu_precision_reference.py:43-45) within its 0.0028 gap, exact rational
  arithmetic for the single-rounding claim, and the C restatement bit for bit;
- bit windows: the literal scalar ``dq`` index arithmetic (exl3_dq.cuh:15-31) and the
  half-rate group form ``dq8_half`` (exl3_dq.cuh:254-285) restated with Python integers,
  against the oracle's funnel and bit-string extractors and the C forms;
- tile map: enumeration from the fragment layouts (ptx_rocm.cuh:11-14, exl3_dq.cuh:153-160);
- Hadamard: ``scipy.linalg.hadamard`` (Sylvester) in float64, exact on integer inputs.
"""
from fractions import Fraction

import numpy as np
import pytest
import scipy.linalg

from oracle import cnative, exl3

RATES = (1, 2, 3, 4, 5, 6, 7, 8, 1.5, 2.5, 3.5)


def _mul1_integer(state):
    # runtime/ds41/cpu_precision_reference.py:43-45 (integer identity of the MUL1 decode)
    product = (int(state) * 0x83DCD12D) & 0xFFFFFFFF
    return sum((product >> bit) & 255 for bit in (0, 8, 16, 24)) - 510


def _random_words(rng, n, K):
    return rng.integers(0, 2**32, size=(n, exl3.tile_words(K)), dtype=np.uint64).astype(np.uint32)


# ---------------------------------------------------------------------------------------------
# Codebook


def test_codebook_against_reference_integer_identity():
    lut = exl3.codebook_lut().astype(np.float64)
    scale = float(np.uint16(0x1EEE).view(np.float16))
    ident = np.array([_mul1_integer(s) for s in range(65536)], dtype=np.float64) * scale
    gap = np.abs(lut - ident)
    assert gap.max() <= 0.0028
    assert gap.max() > 0.0          # the identity is not the fp16 decode itself


def test_codebook_single_rounding_exact_rationals():
    """w = RNE_fp16(h*k + b) with h = 1024 + bytesum, evaluated in exact rationals."""
    k = Fraction(float(np.uint16(0x1EEE).view(np.float16)))
    b = Fraction(float(np.uint16(0xC931).view(np.float16)))
    lut = exl3.codebook_lut()
    by_sum = {}
    for s in range(0, 65536, 37):
        p = (s * 0x83DCD12D) & 0xFFFFFFFF
        bs = (p & 255) + ((p >> 8) & 255) + ((p >> 16) & 255) + (p >> 24)
        exact = (1024 + bs) * k + b
        # round to fp16 by brute force: nearest of the two neighbouring fp16 values, ties to even
        lo = np.float16(float(exact))
        cands = sorted({float(np.nextafter(lo, np.float16(-np.inf))), float(lo),
                        float(np.nextafter(lo, np.float16(np.inf)))}, key=lambda c: (abs(Fraction(c) - exact),
                                                                                   int(np.float16(c).view(np.uint16)) & 1))
        assert float(lut[s]) == cands[0], s
        by_sum.setdefault(bs, float(lut[s]))
        assert by_sum[bs] == float(lut[s])


def test_codebook_closed_form_invariants():
    lut = exl3.codebook_lut().astype(np.float64)
    assert np.isclose(lut.min(), -3.453, atol=1e-3) and np.isclose(lut.max(), 3.348, atol=1e-3)
    assert not np.any(lut == 0.0)
    assert np.all(np.abs(lut) >= 2.0**-14)                      # no subnormals
    assert abs(lut.std() - 1.0) < 0.02
    bs = exl3.mul1_bytesum(np.arange(65536))
    order = np.argsort(bs, kind="stable")
    assert np.all(np.diff(lut[order]) >= 0)                     # monotone in the byte sum


def test_codebook_c_restatement_bit_exact():
    c = cnative.codebook()
    assert np.array_equal(c.view(np.uint16), exl3.codebook_lut().view(np.uint16))


# ---------------------------------------------------------------------------------------------
# Bit windows


def _dq_scalar_state(words, bits, t_offset):
    """exl3_dq.cuh:15-31 with Python integers (integer rates)."""
    b0 = t_offset * bits + bits - 16 + 256 * bits
    b1 = b0 + 16
    i0 = b0 // 32
    i1 = (b1 - 1) // 32
    s0 = (i1 + 1) * 32 - b1
    n = bits * 256 // 32
    a = int(words[i0 % n])
    b = int(words[i1 % n])
    return (((a << 32) | b) >> (s0 & 31)) & 0xFFFF


def _dq8_half_states(words, KA, t_offset):
    """exl3_dq.cuh:254-285 with Python integers: states of positions t_offset..t_offset+7."""
    bits2 = 2 * KA + 1
    nw = 4 * bits2
    gspan = 18 + 3 * KA
    e7 = ((t_offset >> 1) + 4) * bits2 + 128 * bits2
    e3 = e7 - 2 * bits2
    out = []
    for e in (e3, e7):
        hi, lo = (e - 1) // 32, (e - gspan) // 32
        s = (hi + 1) * 32 - e
        a, b = int(words[lo % nw]), int(words[hi % nw])
        w3 = (((a << 32) | b) >> s) & 0xFFFFFFFF
        w2 = w3 >> (KA + 1)
        w1 = w2 >> KA
        w0 = w1 >> (KA + 1)
        out += [w0 & 0xFFFF, w1 & 0xFFFF, w2 & 0xFFFF, w3 & 0xFFFF]
    return out


@pytest.mark.parametrize("K", RATES)
def test_window_extractors_agree_with_reference_index_arithmetic(K):
    rng = np.random.default_rng(int(2 * K) + 11)
    words = _random_words(rng, 6, K)
    funnel = exl3.tile_states_funnel(words, K)
    bitstr = exl3.tile_states_bits(words, K)
    assert np.array_equal(funnel, bitstr)
    for t in range(words.shape[0]):
        if exl3.is_half(K):
            lit = [v for off in range(0, 256, 8) for v in _dq8_half_states(words[t], int(K), off)]
        else:
            lit = [_dq_scalar_state(words[t], int(K), p) for p in range(256)]
        assert np.array_equal(funnel[t], np.array(lit, dtype=np.uint16)), (K, t)


@pytest.mark.parametrize("K", RATES)
def test_window_c_forms(K):
    rng = np.random.default_rng(int(2 * K) + 101)
    words = _random_words(rng, 3, K)
    ref = exl3.tile_states_funnel(words, K)
    for t in range(words.shape[0]):
        assert np.array_equal(cnative.states_scalar(words[t], K), ref[t])
        if K <= 5:
            assert np.array_equal(cnative.states_group8(words[t], K), ref[t])


@pytest.mark.parametrize("K", RATES)
def test_window_geometry(K):
    end = exl3.position_end_bits(K)
    assert end[-1] == 32 * exl3.tile_words(K) == round(256 * K)     # the stream is used up exactly
    steps = np.diff(np.concatenate([[0], end]))
    if exl3.is_half(K):
        assert set(steps[0::2]) == {int(K)} and set(steps[1::2]) == {int(K) + 1}
    else:
        assert set(steps) == {int(K)}


def test_planted_states_round_trip():
    """K=8: each position owns exactly its 16-bit window's low byte pair; plant and read back."""
    rng = np.random.default_rng(5)
    K = 8
    bits = rng.integers(0, 2, size=32 * exl3.tile_words(K), dtype=np.uint8)
    words = exl3.pack_tile_bitstring(bits)
    states = exl3.tile_states_funnel(words[None], K)[0]
    end = exl3.position_end_bits(K)
    for p in (0, 1, 77, 255):
        want = 0
        for i in range(16):
            want = (want << 1) | int(bits[(end[p] - 16 + i) % bits.size])
        assert int(states[p]) == want


# ---------------------------------------------------------------------------------------------
# Tile map and dequant


def test_tile_coords_from_fragment_layout():
    """Lane l holds B fragment b[i] = {B[2t+8i][g], B[2t+8i+1][g]} (g = l/4, t = l%4); its 8
    decoded positions fill f0 = (d0d1, d2d3) for columns 0..7 and f1 = (d4d5, d6d7) for 8..15."""
    kk, nn = exl3.tile_coords()
    want = {}
    for lane in range(32):
        g, t = lane // 4, lane % 4
        for f in range(2):               # f0 / f1
            for i in range(2):           # fragment element b[i]
                for h in range(2):       # low / high half of the half2
                    j = 4 * f + 2 * i + h
                    want[8 * lane + j] = (2 * t + 8 * i + h, g + 8 * f)
    assert [want[p] for p in range(256)] == list(zip(kk.tolist(), nn.tolist()))
    assert len(set(want.values())) == 256


@pytest.mark.parametrize("K", (2, 3, 4, 5, 2.5))
def test_dequant_against_python_loop(K):
    rng = np.random.default_rng(int(2 * K))
    kt, nt = 2, 3
    trellis = rng.integers(-32768, 32768, size=(kt, nt, exl3.tile_u16(K)), dtype=np.int64).astype(np.int16)
    W = exl3.dequant(trellis, K)
    u = trellis.view(np.uint16).astype(np.int64)
    lut = exl3.codebook_lut()
    kk, nn = exl3.tile_coords()
    for a in range(kt):
        for b in range(nt):
            words = [int(u[a, b, 2 * w]) | (int(u[a, b, 2 * w + 1]) << 16) for w in range(exl3.tile_words(K))]
            for p in range(0, 256, 5):
                if exl3.is_half(K):
                    st = _dq8_half_states(words, int(K), p & ~7)[p & 7]
                else:
                    st = _dq_scalar_state(words, int(K), p)
                assert W[16 * a + kk[p], 16 * b + nn[p]] == lut[st]
    assert np.array_equal(cnative.dequant(trellis, K).view(np.uint16), W.view(np.uint16))


# ---------------------------------------------------------------------------------------------
# Hadamard


def test_had128_equals_sylvester():
    rng = np.random.default_rng(3)
    H = scipy.linalg.hadamard(128).astype(np.float64)
    v = rng.standard_normal((16, 256)).astype(np.float32)
    got = exl3.had128(v).astype(np.float64)
    ref = (v.astype(np.float64).reshape(16, 2, 128) @ H.T).reshape(16, 256) * float(exl3.R_SCALE)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # integer inputs: every partial sum is exact, so only the final scale rounds
    vi = rng.integers(-1000, 1000, size=(8, 128)).astype(np.float32)
    exact = (vi.astype(np.float64) @ H.T).astype(np.float32) * exl3.R_SCALE
    assert np.array_equal(exl3.had128(vi), exact)


def test_had128_involution_and_c_form():
    rng = np.random.default_rng(4)
    v = rng.standard_normal((32, 128)).astype(np.float32)
    back = exl3.had128(exl3.had128(v))
    assert np.abs(back - v).max() < 1e-5
    assert np.array_equal(cnative.had128(v), exl3.had128(v))


def test_had128_evaluation_order_is_observable():
    """The fp32 butterfly order matters bit for bit: a different order (bits high to low)
    gives different roundings on random data, so the GPU's bit-exact checks pin the order."""
    rng = np.random.default_rng(9)
    v = rng.standard_normal((64, 128)).astype(np.float32)
    y = v.copy()
    h = 64
    while h >= 1:
        z = y.reshape(-1, 128 // (2 * h), 2, h)
        a, b = z[:, :, 0, :].copy(), z[:, :, 1, :].copy()
        z[:, :, 0, :], z[:, :, 1, :] = a + b, a - b
        y = z.reshape(-1, 128)
        h //= 2
    assert not np.array_equal(y * exl3.R_SCALE, exl3.had128(v))
