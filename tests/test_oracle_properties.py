"""Property tests of the oracle with hypothesis (CPU): the search explores the edge inputs that the
seeded cases may miss (empty calls, one expert, repeated and out-of-range experts, zero routing
weights, ties, signed zeros, subnormals, infinities). Each property is stated independently of
the oracle's own code: the run table against the run-cutting rules (`_check_table`), the top-k
against Python's sort on (key desc, index asc), the Hadamard against its algebra, and the bf16 /
fp16 roundings against torch's casts."""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st
from hypothesis.extra import numpy as hnp

from oracle import coop, exl3
from tests.test_oracle_coop import _check_table

SETTINGS = settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.too_slow])


@st.composite
def routes(draw):
    t = draw(st.integers(0, 24))
    k = draw(st.integers(1, 8))
    E = draw(st.integers(1, 20))
    sel = draw(hnp.arrays(np.int64, (t, k), elements=st.integers(-2, E + 2)))
    rw = draw(hnp.arrays(np.float16, (t, k), elements=st.sampled_from([0.0, -0.0, 0.25, 1.0, -0.5, 6e-8])))
    cap = t + draw(st.integers(0, 3))
    lo = draw(st.integers(-1, E))
    hi = draw(st.integers(max(lo, 0), E + 2)) if lo >= 0 else 0
    return sel, rw, cap, lo, hi


@SETTINGS
@given(routes())
def test_run_table_rules(r):
    """Every active slot once, stably sorted by (local expert, slot), runs cut at expert changes
    and every 8 slots, zeros past the used entries, for any routes (out-of-range experts and zero
    weights inactive, an expert range or none, an empty call)."""
    sel, rw, cap, lo, hi = r
    if lo < 0:
        # without an expert range every non-negative id is a local expert
        sel = np.abs(sel)
        table = coop.reference_table(sel, rw, cap)
        _check_table(sel, rw, table, cap)
    else:
        table = coop.reference_table(sel, rw, cap, lo, hi)
        _check_table(sel, rw, table, cap, lo, hi)


@SETTINGS
@given(hnp.arrays(np.float32, st.integers(1, 40),
                  elements=st.sampled_from([0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 1e-30, -1e-30, 3.0, 3.0000002])),
       st.data())
def test_stable_topk_against_sorting(keys, data):
    """The k largest keys, (key desc, index asc), +0 and -0 equal: the first k of Python's sort."""
    k = data.draw(st.integers(1, keys.size))
    got = coop.stable_topk(keys[None, :], k)[0].tolist()
    want = sorted(range(keys.size), key=lambda i: (-float(keys[i]) if keys[i] != 0 else 0.0, i))[:k]
    assert got == want


finite = st.floats(-1e3, 1e3, allow_nan=False, allow_infinity=False, width=32)


@SETTINGS
@given(hnp.arrays(np.float32, 128, elements=finite), hnp.arrays(np.float32, 128, elements=finite))
def test_had128_algebra(a, b):
    """H128/sqrt(128) is orthogonal and its own inverse, and linear (within fp32 rounding)."""
    ha, hb = exl3.had128(a), exl3.had128(b)
    scale = 1 + float(np.max(np.abs(a))) + float(np.max(np.abs(b)))
    assert np.allclose(exl3.had128(ha), a, atol=1e-5 * scale)
    assert np.allclose(exl3.had128(a + b), ha + hb, atol=1e-5 * scale)
    assert np.isclose(float(np.dot(ha.astype(np.float64), ha)), float(np.dot(a.astype(np.float64), a)),
                      rtol=1e-5, atol=1e-5 * scale * scale)


@SETTINGS
@given(hnp.arrays(np.float32, st.integers(1, 64), elements=st.floats(width=32, allow_nan=False)))
def test_round_bf16_against_torch(v):
    """round_bf16 is torch's fp32 -> bf16 cast (ties to even, overflow to inf, subnormals, -0)."""
    want = torch.from_numpy(v.copy()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(coop.round_bf16(v).view(np.uint32), want.view(np.uint32))


@pytest.mark.filterwarnings("ignore:overflow encountered in cast")   # values past fp16's range go to inf
@SETTINGS
@given(hnp.arrays(np.float32, st.integers(1, 64), elements=st.floats(width=32, allow_nan=False)))
def test_round_fp16_against_torch(v):
    """round_fp16 is the IEEE fp32 -> fp16 cast that torch and the device use."""
    want = torch.from_numpy(v.copy()).to(torch.float16).numpy()
    assert np.array_equal(exl3.round_fp16(v).view(np.uint16), want.view(np.uint16))
