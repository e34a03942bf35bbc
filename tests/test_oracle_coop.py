"""Pins the routing / grouping / expert-math oracle (``oracle/coop.py``) independently.

- router: brute-force sort with the stable key of ``_stable_topk_indices``
  (runtime/ds41/model.py:940-953), the special cases T=1 and all-equal rows, +0 == -0, and the
  portable fp32 score functions against float64 math;
- run table: invariants that characterise ``reference_runs``/``reference_table``
  (runtime/ds41/moe_coop3072.py:64-106): a permutation of the active slots sorted by
  (expert, slot), cuts exactly at expert changes and every 8 slots, run count
  sum(ceil(n_e/8)); plus a hand-worked table;
- expert / layer math: an independent dense float64 formula with the Sylvester matrix of
  ``scipy.linalg.hadamard`` and plain matrix products, the activation semantics of
  K.cuh:115-129 (clamp after SiLU) vs kernels.py:213-217 (clamp before SiLU), and exact
  linearity in the routing weights.
"""
import math

import numpy as np
import pytest
import scipy.linalg

from oracle import coop, exl3, synth

H128 = scipy.linalg.hadamard(128).astype(np.float64) / math.sqrt(128.0)


# ---------------------------------------------------------------------------------------------
# Router


def test_stable_topk_brute_force_with_ties():
    rng = np.random.default_rng(0)
    keys = rng.integers(-3, 4, size=(50, 40)).astype(np.float32)       # many ties
    keys[:, 7] = -0.0
    keys[:, 9] = 0.0
    got = coop.stable_topk(keys, 6)
    for r in range(keys.shape[0]):
        want = sorted(range(40), key=lambda i: (-float(keys[r, i]), i))[:6]
        assert got[r].tolist() == want


def test_router_special_cases():
    z = np.zeros((1, 256), dtype=np.float32)
    idx, w = coop.route(z, 8)
    assert idx.tolist() == [list(range(8))]
    assert np.allclose(w, 1.0 / 8, rtol=1e-6)
    idx, w = coop.route(np.full((3, 64), 0.25, np.float32), 4, "sqrt_softplus", route_scale=1.5)
    assert idx.tolist() == [[0, 1, 2, 3]] * 3
    assert np.allclose(w.sum(-1), 1.5, rtol=1e-6)


def test_router_selection_and_weights():
    rng = np.random.default_rng(1)
    z = rng.standard_normal((16, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    for fn, f64 in (("sigmoid", lambda v: 1 / (1 + np.exp(-v))),
                    ("sqrt_softplus", lambda v: np.sqrt(np.log1p(np.exp(v))))):
        for b in (None, bias):
            idx, w = coop.route(z, 8, fn, b, route_scale=2.5)
            s64 = f64(z.astype(np.float64))
            key = s64 + (0 if b is None else b.astype(np.float64))
            want = np.argsort(-key, axis=-1, kind="stable")[:, :8]
            assert np.array_equal(idx, want)
            g = np.take_along_axis(s64, want, -1)
            assert np.allclose(w, g / g.sum(-1, keepdims=True) * 2.5, rtol=2e-6)


def test_portable_score_functions():
    z = np.linspace(-30, 30, 20001, dtype=np.float32)
    e = coop.exp_f32(z).astype(np.float64)
    assert np.max(np.abs(e / np.exp(z.astype(np.float64)) - 1)) < 4e-7
    s = coop.sigmoid_f32(z).astype(np.float64)
    assert np.max(np.abs(s - 1 / (1 + np.exp(-z.astype(np.float64))))) < 2e-7
    q = coop.sqrt_softplus_f32(z).astype(np.float64)
    q64 = np.sqrt(np.logaddexp(0, z.astype(np.float64)))
    assert np.max(np.abs(q / q64 - 1)) < 5e-7


# ---------------------------------------------------------------------------------------------
# Run table


def _check_table(sel, rw, table, capacity, min_expert=-1, max_expert=0):
    t, k = sel.shape
    ok, local = coop.slot_active(sel, rw, min_expert, max_expert)
    n_runs = int(table[0])
    assert table[1] == 0
    starts = table[2:2 + n_runs + 1]
    n_active = int(ok.sum())
    assert starts[0] == 0 and starts[-1] == n_active and np.all(np.diff(starts) > 0)
    order = table[2 + capacity * k + 1:2 + capacity * k + 1 + n_active]
    # a permutation of the active slots, sorted by (expert, slot)
    act = np.nonzero(ok.reshape(-1))[0]
    assert sorted(order.tolist()) == act.tolist()
    keys = [(int(local.flat[s]), int(s)) for s in order]
    assert keys == sorted(keys)
    # cuts exactly at an expert change and every 8 slots of one expert
    for a, b in zip(starts[:-1], starts[1:]):
        es = {keys[i][0] for i in range(a, b)}
        assert len(es) == 1 and b - a <= coop.ROWS
    counts = np.bincount(local.reshape(-1)[act], minlength=1) if n_active else np.zeros(1, int)
    assert n_runs == int(sum(-(-c // coop.ROWS) for c in counts if c))
    # unused entries stay zero
    assert not np.any(table[2 + n_runs + 1:2 + capacity * k + 1])
    assert not np.any(table[2 + capacity * k + 1 + n_active:])


@pytest.mark.parametrize("seed", range(6))
def test_run_table_invariants(seed):
    rng = np.random.default_rng(seed)
    t, k, E = int(rng.integers(1, 40)), int(rng.integers(1, 9)), int(rng.integers(2, 24))
    sel = np.stack([rng.choice(E, size=k, replace=False) if k <= E else rng.integers(0, E, k) for _ in range(t)])
    rw = rng.standard_normal((t, k)).astype(np.float16)
    rw[rng.random((t, k)) < 0.2] = 0
    cap = t + int(rng.integers(0, 4))
    _check_table(sel, rw, coop.reference_table(sel, rw, cap), cap)
    lo, hi = 1, max(2, E // 2)
    _check_table(sel, rw, coop.reference_table(sel, rw, cap, lo, hi), cap, lo, hi)


def test_run_table_hand_worked():
    # 10 tokens all picking expert 3 in slot 0 and expert 1 in slot 1; slot 1 of token 4 inactive
    sel = np.array([[3, 1]] * 10)
    rw = np.ones((10, 2), np.float16)
    rw[4, 1] = 0
    table = coop.reference_table(sel, rw, capacity=10)
    # expert 1: slots 1,3,5,7,11,13,15,17,19 (9 slots -> runs of 8 + 1); expert 3: 0,2,...,18 (8+2)
    assert table[0] == 4
    assert table[2:7].tolist() == [0, 8, 9, 17, 19]
    order = table[23:23 + 19].tolist()
    assert order == [1, 3, 5, 7, 11, 13, 15, 17, 19, 0, 2, 4, 6, 8, 10, 12, 14, 16, 18]
    assert len(table) == 2 + 2 * 20 + 1


def test_expert_csr_matches_runs():
    rng = np.random.default_rng(7)
    sel = rng.integers(0, 16, size=(20, 4))
    rw = np.ones((20, 4), np.float16)
    off, order = coop.expert_csr(sel, rw, 16)
    flat = [s for _, ss in coop.reference_runs(sel, rw) for s in ss]
    assert order.tolist() == flat
    assert np.array_equal(np.diff(off), np.bincount(sel.reshape(-1), minlength=16))


# ---------------------------------------------------------------------------------------------
# Expert math


def _dense_expert(x16, ew, limit, clamp_after=True):
    """Float64 restatement with explicit matrices; fp16 rounding at the reference's points."""
    f16 = lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float64)
    had = lambda a: (np.asarray(a, np.float64).reshape(-1, 128) @ H128).reshape(np.shape(a))
    x = x16.astype(np.float64)
    Wg, Wu, Wd = (ew.W(p).astype(np.float64) for p in "gud")
    sv = lambda p, q: ew.parts[p][q].astype(np.float64)
    g = had(f16(f16(had(x * sv("g", 1))) @ Wg)) * sv("g", 2)
    u = had(f16(f16(had(x * sv("u", 1))) @ Wu)) * sv("u", 2)
    silu = lambda v: v / (1 + np.exp(-v))
    if clamp_after:
        a = np.minimum(silu(g), limit) * np.clip(u, -limit, limit)
    else:
        a = silu(np.minimum(g, limit)) * np.clip(u, -limit, limit)
    act = f16(had(a * sv("d", 1)))
    return had(act @ Wd) * sv("d", 2)


def _small_expert(rng, H=256, I=128, K=3):
    return synth.expert(rng, H, I, K, svh_scale=1.0 / 16)


def test_coop_expert_against_dense_formula():
    rng = np.random.default_rng(11)
    ew = _small_expert(rng)
    x = (rng.standard_normal((3, 256)) * 2).astype(np.float16)
    got = coop.coop_expert(x, ew, 10.0)
    ref = _dense_expert(x, ew, 10.0)
    assert coop.rel_err_rows(got, ref) < 5e-3


def test_expert_with_its_own_down_rate():
    """Gate/up at 4 bpw, down at 3 bpw (the launcher's K_gu / K_d, exl3_moe_coop.cuh:80-83):
    each projection decodes at its own rate, and the expert matches the dense formula."""
    rng = np.random.default_rng(21)
    ew = synth.expert(rng, 256, 128, 4, svh_scale=1.0 / 16, K_down=3)
    assert ew.parts["g"][0].shape[-1] == 64 and ew.parts["d"][0].shape[-1] == 48
    assert np.array_equal(ew.W("d").view(np.uint16), exl3.dequant(ew.parts["d"][0], 3).view(np.uint16))
    assert np.array_equal(ew.W("g").view(np.uint16), exl3.dequant(ew.parts["g"][0], 4).view(np.uint16))
    x = (rng.standard_normal((2, 256)) * 2).astype(np.float16)
    assert coop.rel_err_rows(coop.coop_expert(x, ew, 10.0), _dense_expert(x, ew, 10.0)) < 5e-3
    assert coop.rel_err_rows(coop.shared_expert(x, ew, 10.0), _dense_expert(x, ew, 10.0, clamp_after=False)) < 1e-2


def test_shared_gate_closed_forms():
    """Gated shared expert (exl3_moe_coop_kernel.cuh:881-903,942-948): y = routed +
    sigmoid(x . w) * shared. w = 0 gives exactly half the shared term; a large positive dot
    gives the ungated layer, a large negative one the routed part alone."""
    rng = np.random.default_rng(22)
    H, I, E, topk = 256, 128, 4, 2
    experts = [_small_expert(rng, H, I) for _ in range(E)]
    shared = _small_expert(rng, H, I)
    x = synth.activations_bf16(rng, 3, H)
    logits = synth.logits_plain(rng, 3, E)
    y0, idx, _, rw = coop.moe_layer(x, logits, experts, shared, topk, 10.0)
    routed = coop.moe_routed(np.asarray(x, np.float32).astype(np.float16), idx, rw, experts, 10.0)
    sh = y0 - routed
    yh, *_ = coop.moe_layer(x, logits, experts, shared, topk, 10.0, shared_gate_w=np.zeros(H, np.float16))
    assert coop.rel_err_rows(yh - routed, 0.5 * sh) < 1e-5
    w = (rng.standard_normal(H) * 0.05).astype(np.float16)
    g = coop.shared_gate(np.asarray(x, np.float32).astype(np.float16), w)
    assert g.shape == (3,) and np.all((g > 0.01) & (g < 0.99))
    t = np.asarray(x, np.float32).astype(np.float16).astype(np.float64) @ w.astype(np.float64)
    assert np.allclose(g, 1 / (1 + np.exp(-t)), rtol=1e-6)
    yg, *_ = coop.moe_layer(x, logits, experts, shared, topk, 10.0, shared_gate_w=w)
    assert coop.rel_err_rows(yg - routed, g[:, None] * sh) < 1e-5
    big = np.full(H, 60.0, np.float16) * np.sign(np.asarray(x, np.float32)[0]).astype(np.float16)
    yb, *_ = coop.moe_layer(x[:1], logits[:1], experts, shared, topk, 10.0, shared_gate_w=big)
    assert coop.rel_err_rows(yb, y0[:1]) < 1e-6
    yn, *_ = coop.moe_layer(x[:1], logits[:1], experts, shared, topk, 10.0, shared_gate_w=-big)
    assert coop.rel_err_rows(yn, routed[:1]) < 1e-6


def test_activation_clamp_semantics():
    g = np.array([30.0, -30.0, 12.0, 0.5], np.float32)
    u = np.array([20.0, 3.0, -15.0, 0.25], np.float32)
    routed = coop.act_gate(g, u, 10.0)                  # min(silu(g), L) * clamp(u)
    shared = coop.swiglu(g, u, 10.0)                    # silu(min(g, L)) * clamp(u)
    silu = lambda v: v / (1 + math.exp(-v))
    assert np.allclose(routed, [10 * 10, silu(-30) * 3, 10 * -10, silu(0.5) * 0.25], rtol=1e-6)
    assert np.allclose(shared, [silu(10) * 10, silu(-30) * 3, silu(10) * -10, silu(0.5) * 0.25], rtol=1e-6)
    assert routed[0] != shared[0]
    assert np.array_equal(coop.act_gate(g, u, 0.0), (coop.silu_f32(g) * u).astype(np.float32))
    # NaN: the routed kernel's fminf/fmaxf return the limit, torch.clamp keeps the NaN
    nan = np.float32("nan")
    assert coop.act_gate(np.array([nan], np.float32), np.array([nan], np.float32), 10.0)[0] == -100.0
    assert np.isnan(coop.swiglu(np.array([nan], np.float32), np.array([1.0], np.float32), 10.0)[0])
    assert np.isnan(coop.swiglu(np.array([1.0], np.float32), np.array([nan], np.float32), 10.0)[0])


def test_moe_routed_linear_in_weights_and_sum_order():
    rng = np.random.default_rng(12)
    experts = [_small_expert(rng) for _ in range(4)]
    x = rng.standard_normal((3, 256)).astype(np.float16)
    sel = np.array([[0, 2], [1, 3], [2, 2]])
    rw = np.array([[0.5, 0.25], [1.0, 0.0], [0.75, 0.125]], np.float16)
    y = coop.moe_routed(x, sel, rw, experts, 10.0)
    y2 = coop.moe_routed(x, sel, (rw * 2).astype(np.float16), experts, 10.0)
    assert np.array_equal(y2, 2 * y)                    # power-of-two scaling is exact
    o = {e: coop.coop_expert(x, experts[e], 10.0) for e in range(4)}
    want = np.stack([0.5 * o[0][0] + 0.25 * o[2][0], 1.0 * o[1][1], 0.75 * o[2][2] + 0.125 * o[2][2]])
    assert coop.rel_err_rows(y, want) < 1e-6
    # EP filter: only local experts [1, 3) contribute, renumbered from 0
    y_ep = coop.moe_routed(x, sel, rw, {0: experts[1], 1: experts[2]}, 10.0, min_expert=1, max_expert=3)
    want_ep = np.stack([0.25 * o[2][0], 1.0 * o[1][1], 0.75 * o[2][2] + 0.125 * o[2][2]])
    assert coop.rel_err_rows(y_ep, want_ep) < 1e-6


def test_exl3_linear_and_shared_expert_against_dense():
    rng = np.random.default_rng(13)
    ew = _small_expert(rng, K=4)
    x = rng.standard_normal((2, 256)).astype(np.float16)
    tr, suh, svh = ew.parts["g"]
    y = coop.exl3_linear(x, tr, suh, svh, 4)
    had = lambda a: (np.asarray(a, np.float64).reshape(-1, 128) @ H128).reshape(np.shape(a))
    ref = had(had(x.astype(np.float64) * suh.astype(np.float64)) @ ew.W("g").astype(np.float64)) * svh
    assert coop.rel_err_rows(y, ref) < 5e-3
    sh = coop.shared_expert(x, ew, 10.0)
    ref_sh = _dense_expert(x, ew, 10.0, clamp_after=False)
    assert coop.rel_err_rows(sh, ref_sh) < 1e-2


def test_rel_err_rows_definition():
    ref = np.array([[1.0, -4.0, 0.0], [0.0, 0.0, 2.0]])
    y = ref + np.array([[0.04, 0.0, 0.0], [0.0, 0.01, 0.0]])
    assert math.isclose(coop.rel_err_rows(y, ref), 0.01)


@pytest.mark.parametrize("rows", [1, 3])
def test_clamp_orders_separate_at_the_test_limit(rows):
    """At the GPU tests' clipping limit (0.75, unit-variance G and U) the reference layer, the
    layer with the routed clamp moved before SiLU, the one with the shared clamp moved after
    SiLU, and the unclamped one are all more than 5x the 1e-2 tolerance apart, so the GPU tests
    that use this limit tell the clamp orders apart."""
    from tests.gpu_helpers import clamp_variants
    H, I, E, topk = 512, 256, 12, 4
    rng = np.random.default_rng(20 + rows)
    experts = [synth.expert(rng, H, I, 4, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, I, 4, 1 / np.sqrt(H))
    x = synth.activations_bf16(rng, rows, H)
    logits = synth.logits_plain(rng, rows, E)
    v = clamp_variants(lambda: coop.moe_layer(x, logits, experts, shared, topk, 0.75)[0])
    for name in ("routed_swapped", "shared_swapped", "unclamped"):
        assert coop.rel_err_rows(v[name], v["ref"]) > 5e-2, name
    # and the limit of 10 used elsewhere never engages at these scales
    v10 = clamp_variants(lambda: coop.moe_layer(x, logits, experts, shared, topk, 10.0)[0])
    assert np.array_equal(v10["unclamped"], v10["ref"])


# ---------------------------------------------------------------------------------------------
# bf16 residual stream: the oracle's helpers against torch's own fp32 -> bf16 cast
# and bf16 add, the operations of model.py:498-499 (``y.to(x.dtype)`` then ``h + y``).


def _bf16_probe_values():
    rng = np.random.default_rng(41)
    u = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 2**16, size=1 << 16, dtype=np.uint64).astype(np.uint32) << 16
    special = [
        hi | 0x8000,                                   # exact ties, even and odd bf16 neighbours
        hi | 0x7FFF, hi | 0x8001,                      # one below / above a tie
        np.arange(0, 1 << 16, dtype=np.uint32) * 131,  # fp32 subnormals and tiny normals
        np.arange(0x7F7F0000, 0x7F800000, 7, dtype=np.uint32),   # near the overflow edge
        np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x00800000, 0x807FFFFF], np.uint32),
    ]
    v = np.concatenate([u, *special]).astype(np.uint32)
    for s in (0, 0x80000000):
        v = np.concatenate([v, v[: 1 << 16] ^ s])
    v = v[(v & 0x7FFFFFFF) <= 0x7F800000]              # finite and +-inf; NaN checked apart
    return v.view(np.float32)


def test_round_bf16_matches_torch_cast():
    torch = pytest.importorskip("torch")
    x = _bf16_probe_values()
    assert x.size >= 1_000_000
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = coop.round_bf16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    nans = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FBFFFFF], np.uint32).view(np.float32)
    assert np.isnan(coop.round_bf16(nans)).all()
    assert np.isnan(torch.from_numpy(nans).to(torch.bfloat16).float().numpy()).all()


def test_residual_add_matches_torch_bf16_add():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(42)
    n = 1 << 19
    h = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * 4).to(torch.bfloat16)
    y = rng.standard_normal(n).astype(np.float32) * np.float32(2.0) ** rng.integers(-12, 6, n).astype(np.float32)
    # ties of the final rounding: y a bf16 value that lands h + y exactly between neighbours
    y[:4096] = (h[:4096].float().numpy().view(np.uint32) & 0xFFFF0000).view(np.float32) * np.float32(2.0**-8)
    want = (h + torch.from_numpy(y).to(torch.bfloat16)).float().numpy()
    got = coop.residual_add(h.float().numpy(), y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_layer_stack_one_layer_is_residual_add_of_the_layer():
    H, I, E, topk, K = 256, 128, 6, 2, 3
    rng = np.random.default_rng(43)
    experts = [synth.expert(rng, H, I, K, 1 / np.sqrt(H)) for _ in range(E)]
    shared = synth.expert(rng, H, I, K, 1 / np.sqrt(H))
    h = coop.round_bf16(rng.standard_normal((3, H)).astype(np.float32))
    logits = [synth.logits_plain(rng, 3, E)]
    got = coop.layer_stack(h, logits, [(experts, shared)], topk, 10.0)
    y = coop.moe_layer(h, logits[0], experts, shared, topk, 10.0)[0]
    assert np.array_equal(got, coop.residual_add(h, y))
    # two layers: the second layer routes on its own logits and reads the first's output
    logits2 = logits + [synth.logits_plain(rng, 3, E)]
    got2 = coop.layer_stack(h, logits2, [(experts, shared)] * 2, topk, 10.0)
    y2 = coop.moe_layer(got, logits2[1], experts, shared, topk, 10.0)[0]
    assert np.array_equal(got2, coop.residual_add(got, y2))
