"""Routing, slot grouping and the coop expert math: CPU restatement (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference files (abbreviations as in ``oracle/exl3.py``; ``ds41/`` = runtime/ds41/):

- router: ``ds41/model.py:404-416`` (``Block.route``), tie rule ``ds41/model.py:940-953``
- slot activity: ``K.cuh:200-223`` (``slot_info``)
- run table: ``ds41/moe_coop3072.py:45-106`` (``sort_key``, ``reference_runs``,
  ``reference_table``), device form ``csrc/moe_coop3072/prepare_runs.cuh:8-66``
- routed expert: ``K.cuh:613-629`` (input rotation), ``K.cuh:340-544`` (GEMV tile, fp16
  output for gate/up, fp32 for down), ``K.cuh:758-806`` (gate/up epilogue),
  ``K.cuh:115-129`` (activation), ``K.cuh:860-962`` (slot reduction)
- shared expert: ``ds41/model.py:418-452`` with ``ds41/kernels.py:213-217`` (``swiglu``)
  and the EXL3 linear of ``vendor/quant/exl3_gemv_kernel.cuh:217-234,463-490`` with
  ``hadamard_inner.cuh:93-147``
- layer: ``ds41/model.py:454-499`` (``Block.experts``)

Rounding points follow the reference; the GEMV sums are exact (float64) where the
reference accumulates in fp16 MMAs folded into fp32, so only the tolerance-checked
outputs differ from the reference's device arithmetic.

Pinning (tests/test_oracle_coop.py): the run table is checked against invariants that
characterise it independently (a permutation of the active slots sorted by
(expert, slot); cuts exactly at expert changes and every 8 slots of an expert; run
count = sum of ceil(n_e/8)) and brute force on tiny inputs; the router against
``argsort`` with the stable key and the special cases of the survey (T=1, all-equal
logits -> indices 0..k-1); the expert and layer math against an independent dense
float64 formula built from ``scipy.linalg.hadamard`` and plain matrix products.
"""
from __future__ import annotations

import math

import numpy as np

from . import exl3

ROWS = 8            # slots of one expert per run (K.cuh:40)
F32 = np.float32


# ----------------------------------------------------------------------------------------------
# Portable fp32 elementary functions (mul/add only, no fused operations), mirrored operation
# for operation by the HIP router so that scores and selection keys agree bit for bit.

_LOG2E = F32(1.4426950408889634)
_LN2_HI = F32(0.693145751953125)          # 16 significant bits: n * _LN2_HI is exact for |n| < 256
_LN2_LO = F32(1.428606765330187e-06)
_EXP_COEF = [F32(1.0 / math.factorial(i)) for i in range(8)]


def exp_f32(x):
    """e^x by Cody-Waite reduction x = n ln2 + r and the degree-7 Taylor polynomial of e^r."""
    x = np.clip(np.asarray(x, dtype=F32), F32(-87.0), F32(88.0))
    n = np.rint((x * _LOG2E).astype(F32)).astype(F32)
    r = ((x - (n * _LN2_HI).astype(F32)).astype(F32) - (n * _LN2_LO).astype(F32)).astype(F32)
    p = _EXP_COEF[7]
    for c in _EXP_COEF[6::-1]:
        p = (p * r).astype(F32)
        p = (p + c).astype(F32)
    return np.ldexp(p, n.astype(np.int32)).astype(F32)


def log1p_f32(u):
    """log(1+u) for u in [0, 1]: 2 atanh(s), s = u/(2+u) <= 1/3, odd series to s^15."""
    u = np.asarray(u, dtype=F32)
    s = (u / (F32(2.0) + u)).astype(F32)
    s2 = (s * s).astype(F32)
    p = F32(1.0 / 15.0)
    for d in (13.0, 11.0, 9.0, 7.0, 5.0, 3.0, 1.0):
        p = (p * s2).astype(F32)
        p = (p + F32(1.0 / d)).astype(F32)
    return (F32(2.0) * (s * p).astype(F32)).astype(F32)


def sigmoid_f32(z):
    z = np.asarray(z, dtype=F32)
    return (F32(1.0) / (F32(1.0) + exp_f32(-z))).astype(F32)


def sqrt_softplus_f32(z):
    """sqrt(softplus(z)) = sqrt(max(z,0) + log1p(exp(-|z|))) (model.py:409-410)."""
    z = np.asarray(z, dtype=F32)
    sp = (np.maximum(z, F32(0.0)) + log1p_f32(exp_f32(-np.abs(z)))).astype(F32)
    return np.sqrt(sp).astype(F32)


SCORE_FNS = {"sigmoid": sigmoid_f32, "sqrt_softplus": sqrt_softplus_f32}


def stable_topk(keys, k):
    """Indices of the k largest keys per row, (key desc, index asc); +0 and -0 compare equal.

    This is the ``_stable_topk_indices`` rule (model.py:940-953) with the slots ordered by
    descending key, as ``torch.topk(sorted=True)`` orders ``Block.route``'s result.
    """
    keys = np.asarray(keys, dtype=F32)
    keys = np.where(keys == 0, F32(0.0), keys)
    order = np.lexsort((np.broadcast_to(np.arange(keys.shape[-1]), keys.shape), -keys.astype(np.float64)), axis=-1)
    return order[..., :k].astype(np.int64)


def route(logits, topk: int, score_fn: str = "sigmoid", sel_bias=None, route_scale: float = 1.0):
    """Router: ``idx = topk(score(z) + bias)``, ``w = score(z)[idx] / (sum + 1e-20) * scale``.

    model.py:404-416 with the score function selectable (the reference model uses
    sqrt-softplus; the DeepSeek-V3 configurations use sigmoid). The sum runs over the slots
    in order in fp32. Without a selection bias and with a monotone score the selection is
    made on the logits themselves.
    """
    z = np.asarray(logits, dtype=F32)
    score = SCORE_FNS[score_fn](z)
    if sel_bias is None:
        key = z if score_fn == "sigmoid" else score
    else:
        key = (score + np.asarray(sel_bias, dtype=F32)).astype(F32)
    idx = stable_topk(key, topk)
    s = np.take_along_axis(score, idx, axis=-1)
    tot = np.zeros(s.shape[:-1], dtype=F32)
    for j in range(topk):
        tot = (tot + s[..., j]).astype(F32)
    w = (s / (tot + F32(1e-20))[..., None]).astype(F32)
    w = (w * F32(route_scale)).astype(F32)
    return idx, w


# ----------------------------------------------------------------------------------------------
# Slot activity and run table


def slot_active(sel, rw_fp16, min_expert=-1, max_expert=0):
    """K.cuh:208-223: inactive iff fp16 weight == 0, or the expert is outside the local range."""
    sel = np.asarray(sel, dtype=np.int64)
    ok = np.asarray(rw_fp16, dtype=np.float16).astype(np.float32) != 0
    local = sel.copy()
    if min_expert >= 0:
        ok = ok & (sel >= min_expert) & (sel < max_expert)
        local = sel - min_expert
    return ok, np.where(ok, local, 0)


def reference_runs(sel, rw_fp16=None, min_expert=-1, max_expert=0, rows_per_run=ROWS):
    """moe_coop3072.py:64-83: active slots sorted by (expert, slot), cut at an expert change
    or every ``rows_per_run`` slots of one expert. Returns a list of (expert, [slots])."""
    sel = np.asarray(sel, dtype=np.int64)
    t, k = sel.shape
    if rw_fp16 is None:
        rw_fp16 = np.ones((t, k), dtype=np.float16)
    ok, local = slot_active(sel, rw_fp16, min_expert, max_expert)
    active = sorted((int(local.flat[s]), s) for s in range(t * k) if ok.flat[s])
    runs = []
    for e, s in active:
        if not runs or runs[-1][0] != e or len(runs[-1][1]) == rows_per_run:
            runs.append((e, []))
        runs[-1][1].append(s)
    return runs


def reference_table(sel, rw_fp16=None, capacity=None, min_expert=-1, max_expert=0):
    """moe_coop3072.py:86-106 generalised to any top-k: int32
    ``[n_runs, 0, run_start[0..cap*topk], order[cap*topk]]`` with unused entries zero."""
    sel = np.asarray(sel, dtype=np.int64)
    t, k = sel.shape
    capacity = t if capacity is None else capacity
    if t > capacity:
        raise ValueError("route rows exceed table capacity")
    slots_max = capacity * k
    runs = reference_runs(sel, rw_fp16, min_expert, max_expert)
    table = np.zeros(2 + 2 * slots_max + 1, dtype=np.int32)
    table[0] = len(runs)
    order_off = 2 + slots_max + 1
    pos = 0
    for number, (_, slots) in enumerate(runs):
        table[2 + number] = pos
        for s in slots:
            table[order_off + pos] = s
            pos += 1
    table[2 + len(runs)] = pos
    return table


def expert_csr(sel, rw_fp16, n_experts, min_expert=-1, max_expert=0):
    """Per-expert slot lists in (expert, slot) order: ``offsets[E+1]``, ``order[n_active]``.

    Same order as the run table's ``order``; the runs are these lists cut every 8 slots.
    """
    ok, local = slot_active(sel, rw_fp16, min_expert, max_expert)
    flat_ok = ok.reshape(-1)
    flat_e = local.reshape(-1)
    slots = np.nonzero(flat_ok)[0]
    order = slots[np.lexsort((slots, flat_e[slots]))]
    counts = np.bincount(flat_e[slots], minlength=n_experts)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return offsets, order.astype(np.int32)


# ----------------------------------------------------------------------------------------------
# Expert math


def dequant_fast(trellis, K):
    """Dequantize with the scalar C restatement when it is built (tests pin it to the numpy
    form bit for bit), else with numpy."""
    try:
        from . import cnative
        return cnative.dequant(trellis, K)
    except (OSError, ImportError):
        return exl3.dequant(trellis, K)


class ExpertWeights:
    """One expert's three EXL3 projections (gate, up: [H -> I]; down: [I -> H]).

    ``trellis`` int16 [in/16, out/16, T], ``suh`` fp16 [in], ``svh`` fp16 [out], rate ``K``
    (gate and up; the reference launcher takes one rate for both, exl3_moe_coop.cuh:80-83) and
    ``K_down`` for the down projection (default: ``K``). Decoded fp16 matrices are cached on
    first use.
    """

    def __init__(self, g, u, d, K, K_down=None):
        self.parts = {"g": g, "u": u, "d": d}     # each (trellis, suh, svh)
        self.K = float(K)
        self.K_down = float(K if K_down is None else K_down)
        self._dec = {}

    def rate(self, p):
        return self.K_down if p == "d" else self.K

    def W(self, p):
        if p not in self._dec:
            self._dec[p] = dequant_fast(self.parts[p][0], self.rate(p))
        return self._dec[p]

    def suh(self, p):
        return self.parts[p][1]

    def svh(self, p):
        return self.parts[p][2]


def _f32(a):
    return np.asarray(a, dtype=np.float32)


def rotate_input(x_fp16, suh_fp16):
    """K.cuh:613-629: ``fp16(H128(float(x) * float(suh)))``, zero-padded to len(suh)."""
    x = _f32(np.asarray(x_fp16, dtype=np.float16))
    hi = len(suh_fp16)
    if x.shape[-1] < hi:
        x = np.concatenate([x, np.zeros(x.shape[:-1] + (hi - x.shape[-1],), np.float32)], axis=-1)
    v = (x * _f32(suh_fp16)).astype(np.float32)
    return exl3.round_fp16(exl3.had128(v))


def gemv_exact(a_fp16, W_fp16):
    return np.asarray(a_fp16, dtype=np.float64) @ np.asarray(W_fp16, dtype=np.float64)


def silu_f32(g):
    g64 = np.asarray(g, dtype=np.float64)
    return (g64 / (1.0 + np.exp(-g64))).astype(np.float32)


def act_gate(g, u, limit):
    """K.cuh:115-129 (SiLU, gated): ``min(silu(g), L) * clamp(u, -L, L)`` when L != 0, with the
    kernel's fminf/fmaxf, which return the other operand when one is NaN (np.fmin/np.fmax)."""
    x = silu_f32(g)
    u = _f32(u)
    if limit != 0:
        u = np.fmin(np.fmax(u, F32(-limit)), F32(limit)).astype(np.float32)
        x = np.fmin(x, F32(limit)).astype(np.float32)
    return (x * u).astype(np.float32)


def coop_expert(x_fp16, ew: ExpertWeights, limit: float):
    """Routed expert for rows of x: fp32 ``[R, H]`` before the routing weight (A.6 steps 1-7)."""
    xg = rotate_input(x_fp16, ew.suh("g"))
    xu = rotate_input(x_fp16, ew.suh("u"))
    gu_g = exl3.round_fp16(gemv_exact(xg, ew.W("g")))            # gu_f32 = false
    gu_u = exl3.round_fp16(gemv_exact(xu, ew.W("u")))
    G = (exl3.had128(_f32(gu_g)) * _f32(ew.svh("g"))).astype(np.float32)
    U = (exl3.had128(_f32(gu_u)) * _f32(ew.svh("u"))).astype(np.float32)
    a = act_gate(G, U, limit)
    a = (a * _f32(ew.suh("d"))).astype(np.float32)
    act = exl3.round_fp16(exl3.had128(a))
    d = gemv_exact(act, ew.W("d")).astype(np.float32)            # c_f32 = true
    return (exl3.had128(d) * _f32(ew.svh("d"))).astype(np.float32)


def moe_routed(x_fp16, sel, rw_fp16, experts, limit, min_expert=-1, max_expert=0):
    """K.cuh:860-962: per token, ``sum_k w_k * o_{r,k}`` over active slots in slot order (fp32).

    ``experts``: sequence or dict of ExpertWeights indexed by local expert.
    """
    x = np.asarray(x_fp16, dtype=np.float16)
    sel = np.asarray(sel, dtype=np.int64)
    rw = np.asarray(rw_fp16, dtype=np.float16)
    t, k = sel.shape
    ok, local = slot_active(sel, rw, min_expert, max_expert)
    hout = x.shape[1]
    out = np.zeros((t, hout), dtype=np.float32)
    cache = {}
    for e in sorted(set(int(v) for v in local[ok])):
        rows = sorted({r for r in range(t) for j in range(k) if ok[r, j] and local[r, j] == e})
        o = coop_expert(x[rows], experts[e], limit)
        for i, r in enumerate(rows):
            cache[(r, e)] = o[i]
    for r in range(t):
        acc = np.zeros(hout, dtype=np.float32)
        for j in range(k):
            if not ok[r, j]:
                continue
            w = F32(float(rw[r, j]))
            acc = (acc + (w * cache[(r, int(local[r, j]))]).astype(np.float32)).astype(np.float32)
        out[r] = acc
    return out


def exl3_linear(x_fp16, trellis, suh, svh, K, W=None):
    """Single EXL3 linear with fp16 output (exl3_gemv_kernel.cuh:217-234,463-490).

    Input: ``fp16(x * suh)`` (fp16 product, hadamard_inner.cuh:109-115), Hadamard in fp32,
    fp16; GEMV to fp16; output Hadamard in fp32 to fp16, then ``fp16(y * svh)``
    (hadamard_inner.cuh:133-143).
    """
    x = np.asarray(x_fp16, dtype=np.float16)
    v = (_f32(x) * _f32(suh)).astype(np.float16)
    xr = exl3.round_fp16(exl3.had128(_f32(v)))
    Wd = exl3.dequant(trellis, K) if W is None else W
    c = exl3.round_fp16(gemv_exact(xr, Wd))
    y = exl3.round_fp16(exl3.had128(_f32(c)))
    return (_f32(y) * _f32(svh)).astype(np.float16)


def swiglu(gate, up, limit):
    """kernels.py:213-217: clamp the gate from above BEFORE SiLU, the up symmetrically, with
    torch.clamp's semantics (a NaN stays NaN: np.clip / np.minimum)."""
    gate = _f32(gate)
    up = _f32(up)
    if limit > 0:
        up = np.clip(up, F32(-limit), F32(limit)).astype(np.float32)
        gate = np.minimum(gate, F32(limit)).astype(np.float32)
    return (silu_f32(gate) * up).astype(np.float32)


def shared_expert(x_fp16, ew: ExpertWeights, limit):
    """model.py:450-452: gate/up EXL3 linears, fp32 swiglu, fp16, down linear, fp32."""
    gate = exl3_linear(x_fp16, *ew.parts["g"], ew.rate("g"), W=ew.W("g"))
    up = exl3_linear(x_fp16, *ew.parts["u"], ew.rate("u"), W=ew.W("u"))
    mid = swiglu(gate, up, limit).astype(np.float16)
    return _f32(exl3_linear(mid, *ew.parts["d"], ew.rate("d"), W=ew.W("d")))


def shared_gate(x_fp16, gate_w_fp16):
    """exl3_moe_coop_kernel.cuh:881-903: the gated shared expert's per-row scale
    sigmoid(x_row . w), the dot in fp32 over fp16 values (the kernel's reduction order and
    __expf are not reproduced: held to tolerance)."""
    x = _f32(np.asarray(x_fp16, dtype=np.float16)).astype(np.float64)
    w = _f32(np.asarray(gate_w_fp16, dtype=np.float16)).astype(np.float64)
    t = x @ w
    return (1.0 / (1.0 + np.exp(-t))).astype(np.float32)


def moe_layer(x, logits, experts, shared, topk, limit, score_fn="sigmoid", sel_bias=None,
              route_scale=1.0, shared_gate_w=None):
    """Block.experts (model.py:454-499) for one layer, routed from given logits.

    Returns (y fp32 [T,H] = routed + shared, idx, w fp32, rw fp16). The caller casts y to
    the activation dtype (model.py:499). With ``shared_gate_w`` the shared term is
    sigmoid(x . w) * shared (exl3_moe_coop_kernel.cuh:942-948).
    """
    xh = np.asarray(x, dtype=np.float32).astype(np.float16)
    idx, w = route(logits, topk, score_fn, sel_bias, route_scale)
    rw = w.astype(np.float16)
    y = moe_routed(xh, idx, rw, experts, limit)
    if shared is not None:
        sh = shared_expert(xh, shared, limit)
        if shared_gate_w is not None:
            sh = (shared_gate(xh, shared_gate_w)[:, None] * sh).astype(np.float32)
        y = (y + sh).astype(np.float32)
    return y, idx, w, rw


def round_bf16(v):
    """fp32 -> nearest bf16 (ties to even; overflow to +-inf), returned as float32 values.
    A NaN stays a NaN (quieted), as torch's ``.to(torch.bfloat16)`` keeps it."""
    x = np.ascontiguousarray(np.asarray(v, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, ((u >> 16) | 0x40) << 16, r)
    return r.astype(np.uint32).view(np.float32)


def residual_add(h_bf16, y):
    """model.py:499 then the residual: ``h + y.to(bf16)`` in bf16 (fp32 add, one rounding)."""
    return round_bf16(np.asarray(h_bf16, np.float32) + round_bf16(y))


def layer_stack(h_bf16, logits, layers, topk, limit, score_fn="sigmoid"):
    """Config 5: MoE layers applied in turn with a bf16 residual stream.

    ``logits[l]`` routes layer l (independent of h, as the configuration draws them);
    ``layers[l] = (experts, shared)``. Returns the final bf16 stream (as float32 values).
    """
    h = round_bf16(h_bf16)
    for l, (experts, shared) in enumerate(layers):
        y, _, _, _ = moe_layer(h, logits[l], experts, shared, topk, limit, score_fn)
        h = residual_add(h, y)
    return h


def rel_err_rows(y, ref):
    """max_r ( max|y_r - ref_r| / max|ref_r| ): the tolerance metric for layer outputs."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.abs(y - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-30)
    return float((num / den).max())
