"""PyTorch-CPU restatement of the MoE layer: the CPU baseline timed by bench.py.

TEST/BASELINE INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). The reference has no PyTorch
CPU implementation of this path (runtime/ds41/cpu_experts.py calls an absent native library
with int8 activations), so the baseline restates the reference math with torch CPU ops:

1. MUL1 LUT decode of every touched projection (states by funnel shifts, exl3_dq.cuh:15-31;
   codebook.cuh:86-99) into fp32 W;
2. 128-point Hadamard rotations as ``[.., 128] @ H128`` (Sylvester, scaled 1/sqrt(128));
3. fp32 ``torch.matmul`` GEMVs;
4. SwiGLU with the coop clamp (exl3_moe_coop_kernel.cuh:115-129) for routed experts and the
   swiglu clamp (kernels.py:213-217) for the shared expert;
5. the weighted sum over slots in slot order plus the shared expert.

Numerically it skips the fp16 rounding points (it is a throughput baseline, not the parity
oracle; ``oracle.coop`` is the parity oracle).
"""
from __future__ import annotations

import numpy as np
import torch

from . import exl3

_H128 = None


def h128() -> torch.Tensor:
    global _H128
    if _H128 is None:
        h = np.array([[1.0]])
        while h.shape[0] < 128:
            h = np.block([[h, h], [h, -h]])
        _H128 = torch.from_numpy(h / np.sqrt(128.0)).float()
    return _H128


def rotate(v: torch.Tensor) -> torch.Tensor:
    """Hadamard over 128-chunks of the last axis (H128 is symmetric)."""
    shp = v.shape
    return (v.reshape(-1, 128) @ h128()).reshape(shp)


class Decoder:
    """Vectorised state extraction + LUT decode for one rate."""

    def __init__(self, K: float):
        i_hi, i_lo, s = exl3.window_plan(K)
        self.i_hi = torch.from_numpy(i_hi)
        self.i_lo = torch.from_numpy(i_lo)
        self.s = torch.from_numpy(s)
        self.lut = torch.from_numpy(exl3.codebook_lut().astype(np.float32))
        kk, nn = exl3.tile_coords()
        self.kk = torch.from_numpy(kk)
        self.nn = torch.from_numpy(nn)

    def dequant(self, trellis: torch.Tensor) -> torch.Tensor:
        """int16 ``[kt, nt, T]`` -> fp32 ``W[kt*16, nt*16]``."""
        kt, nt, t16 = trellis.shape
        u = trellis.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF   # little-endian word view
        hi = u.index_select(2, self.i_hi)
        lo = u.index_select(2, self.i_lo)
        states = ((hi << 32) | lo) >> self.s
        states = states & 0xFFFF
        vals = self.lut[states]                                                   # [kt, nt, 256]
        tiles = torch.empty(kt, nt, 16, 16)
        tiles[:, :, self.kk, self.nn] = vals
        return tiles.permute(0, 2, 1, 3).reshape(kt * 16, nt * 16)


def linear_forward(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                   dec: Decoder) -> torch.Tensor:
    """One EXL3 linear (ELinear.forward, exl3_linear.py:97-131), fp32: H(H(x*suh) @ W) * svh."""
    return rotate(rotate(x * suh.float()) @ dec.dequant(trellis)) * svh.float()


def expert_forward(x: torch.Tensor, parts, dec: Decoder, limit: float, shared: bool) -> torch.Tensor:
    """x fp32 [R, H]; parts = ((trellis, suh, svh) for g, u, d) as CPU tensors."""
    outs = []
    for p in range(2):
        tr, suh, svh = parts[p]
        xr = rotate(x * suh.float())
        outs.append(rotate(xr @ dec.dequant(tr)) * svh.float())
    g, u = outs
    if limit > 0:
        u = u.clamp(-limit, limit)
        if shared:
            g = g.clamp(max=limit)
    a = torch.nn.functional.silu(g)
    if limit > 0 and not shared:
        a = a.clamp(max=limit)
    a = a * u
    tr, suh, svh = parts[2]
    ar = rotate(a * suh.float())
    return rotate(ar @ dec.dequant(tr)) * svh.float()


def route_sigmoid(logits: torch.Tensor, topk: int, route_scale: float = 1.0):
    """Block.route with sigmoid scores (model.py:404-416 with the DeepSeek-V3 score): top-k of
    the logits (sigmoid is monotone), weights normalised over the picks and scaled."""
    z, idx = torch.topk(logits, topk, dim=-1)
    s = torch.sigmoid(z)
    return idx, s / (s.sum(-1, keepdim=True) + 1e-20) * route_scale


def moe_layer(x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, experts, shared, dec, limit: float):
    """Routed slots in slot order plus the shared expert; x fp32 [T, H]. ``dec``: one Decoder for
    every expert, or a dict of Decoders by expert index with the shared expert's under -1."""
    dec_of = (lambda e: dec[e]) if isinstance(dec, dict) else (lambda e: dec)
    t, k = idx.shape
    out = torch.zeros_like(x)
    cache = {}
    for e in sorted(set(idx.reshape(-1).tolist())):
        rows = [r for r in range(t) if e in idx[r].tolist()]
        cache[e] = (rows, expert_forward(x[rows], experts[e], dec_of(e), limit, False))
    for r in range(t):
        for j in range(k):
            e = int(idx[r, j])
            rows, o = cache[e]
            out[r] += w[r, j] * o[rows.index(r)]
    if shared is not None:
        out += expert_forward(x, shared, dec_of(-1), limit, True)
    return out
