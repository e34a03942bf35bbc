"""Writes ``tests/golden/evamx_golden.npz``: small input/output vectors of every function on the
path, produced by the CPU restatement (``oracle/``) after its pinning tests pass.

The reference holds no golden vectors for this path (its tests omit the MoE kernels), so these
fixtures freeze the pinned oracle's outputs: the CPU suite checks that the oracle still
reproduces them, and the GPU suite checks the HIP kernels against them without running the
oracle. Regenerate with ``python tests/golden/make_golden.py`` (deterministic, seeded).

Contents (prefix: meaning):
  dq_K<r>_*     trellis int16 [2,3,T] -> states [2,3,256] uint16, W fp16 [32,48]    (per rate r)
  had_*         v fp32 [4,256] -> had128(v)
  route_<fn>_*  logits [6,64] (+ bias) -> idx int64 [6,4], w fp32 [6,4]
  runs_*        sel int64 [12,4], rw fp16 -> reference table int32 (capacity 12)
  layer_*       a small MoE layer: H=128, I=128, 6 routed experts (K=2, 3), top-2, 3 tokens,
                bf16 x, fp32 logits, shared expert K=4, limit 10 -> y fp32 [3,128], idx, rw
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import coop, exl3, synth  # noqa: E402

OUT = os.path.join(HERE, "evamx_golden.npz")
RATES = (2, 2.5, 3, 4, 5)
LAYER = dict(H=128, I=128, E=6, topk=2, T=3, limit=10.0, shared_K=4)


def rate_tag(K):
    return str(K).replace(".", "p")


def build():
    d = {}
    rng = np.random.default_rng(20261201)
    for K in RATES:
        tr = rng.integers(-32768, 32768, size=(2, 3, exl3.tile_u16(K)), dtype=np.int16)
        t = rate_tag(K)
        d[f"dq_K{t}_trellis"] = tr
        d[f"dq_K{t}_states"] = exl3.trellis_states(tr, K)
        d[f"dq_K{t}_W"] = exl3.dequant(tr, K)
    v = rng.standard_normal((4, 256)).astype(np.float32)
    d["had_v"], d["had_y"] = v, exl3.had128(v)
    z = rng.standard_normal((6, 64)).astype(np.float32)
    z[2] = 0.5                                                    # all-equal row
    bias = (rng.standard_normal(64) * 0.1).astype(np.float32)
    d["route_logits"], d["route_bias"] = z, bias
    for fn in ("sigmoid", "sqrt_softplus"):
        idx, w = coop.route(z, 4, fn, bias if fn == "sqrt_softplus" else None, route_scale=2.5)
        d[f"route_{fn}_idx"], d[f"route_{fn}_w"] = idx, w
    sel = np.stack([rng.choice(10, size=4, replace=False) for _ in range(12)]).astype(np.int64)
    rw = rng.uniform(0.1, 1.0, size=(12, 4)).astype(np.float16)
    rw[rng.random((12, 4)) < 0.25] = 0
    d["runs_sel"], d["runs_rw"] = sel, rw
    d["runs_table"] = coop.reference_table(sel, rw, capacity=12)
    L = LAYER
    experts = [synth.expert(rng, L["H"], L["I"], 2 + (e % 2), svh_scale=1.0 / np.sqrt(L["H"])) for e in range(L["E"])]
    shared = synth.expert(rng, L["H"], L["I"], L["shared_K"], svh_scale=1.0 / np.sqrt(L["H"]))
    x = synth.activations_bf16(rng, L["T"], L["H"])
    logits = synth.logits_plain(rng, L["T"], L["E"])
    y, idx, w, rwl = coop.moe_layer(x, logits, experts, shared, L["topk"], L["limit"])
    for e, ew in enumerate(experts + [shared]):
        tag = "shared" if e == L["E"] else f"e{e}"
        d[f"layer_{tag}_K"] = np.array(ew.K)
        for p in "gud":
            tr, suh, svh = ew.parts[p]
            d[f"layer_{tag}_{p}_trellis"], d[f"layer_{tag}_{p}_suh"], d[f"layer_{tag}_{p}_svh"] = tr, suh, svh
    d["layer_x"], d["layer_logits"] = x, logits
    d["layer_y"], d["layer_idx"], d["layer_rw"] = y, idx, rwl
    return d


def load():
    """The fixture as a dict of arrays (no pickled objects)."""
    with np.load(OUT, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def layer_experts(g):
    """(routed experts, shared expert) of the fixture's layer as oracle ExpertWeights."""
    def ew(tag):
        parts = [tuple(g[f"layer_{tag}_{p}_{n}"] for n in ("trellis", "suh", "svh")) for p in "gud"]
        return coop.ExpertWeights(*parts, K=float(g[f"layer_{tag}_K"]))
    return [ew(f"e{e}") for e in range(LAYER["E"])], ew("shared")


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(OUT, os.path.getsize(OUT), "bytes")
