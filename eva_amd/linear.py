"""Drop-in EXL3 linear: ``ELinear`` / ``build_linear`` of runtime/ds41/exl3_linear.py:64-154,
forwarding to evamx_exl3_linear (fp16 in, fp16 out, the reference's rounding points).

Calls of up to 16 rows take the decode GEMV; larger calls take the MFMA path (the reference
likewise runs small batches row by row and hands larger ones to its GEMM, exl3_linear.py:106-128).
Within each path a row's result is independent of how many rows share the call (the k-split and
the per-row accumulation order depend only on in/out): the batch invariance the reference's
strict small-row mode obtains by running rows one at a time.
"""
from __future__ import annotations

import torch

from . import ops


class ELinear:
    def __init__(self, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor):
        if trellis.ndim != 3 or trellis.dtype != torch.int16:
            raise ValueError("trellis must be int16 [in/16, out/16, 16*K]")
        self.trellis, self.suh, self.svh = trellis, suh, svh
        self.in_features = suh.shape[0]
        self.out_features = svh.shape[0]
        self.k = trellis.shape[-1] / 16
        if trellis.shape[0] * 16 != self.in_features or trellis.shape[1] * 16 != self.out_features:
            raise ValueError("trellis tiles disagree with suh/svh lengths")
        if self.k not in (1.5, 2, 2.5, 3, 3.5, 4, 5):
            raise ValueError(f"EXL3 linear supports 1.5..4 bits in steps of 0.5 and 5 bits, got {self.k}")
        self._ws = None

    def _workspace(self, rows):
        need = ops.lib().evamx_exl3_linear_workspace_bytes(rows, self.in_features, self.out_features)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.trellis.device)
        return self._ws

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, shape[-1]).to(torch.float16).contiguous()
        if flat.shape[-1] != self.in_features:
            raise ValueError("input width differs from the EXL3 metadata")
        y = torch.empty(flat.shape[0], self.out_features, dtype=torch.float16, device=flat.device)
        ops.exl3_linear(flat, self.trellis, self.suh, self.svh, self.k, out=y, workspace=self._workspace(flat.shape[0]))
        return y.reshape(*shape[:-1], self.out_features)

    __call__ = forward


def build_linear(suh, svh, trellis, mul1=None, device: str = "cuda") -> ELinear:
    """exl3_linear.py:134-154. ``mul1`` only marks the MUL1 codebook, the only one supported."""
    suh = suh.to(device=device, dtype=torch.float16).contiguous()
    svh = svh.to(device=device, dtype=torch.float16).contiguous()
    trellis = trellis.to(device=device, dtype=torch.int16).contiguous()
    return ELinear(trellis, suh, svh)
