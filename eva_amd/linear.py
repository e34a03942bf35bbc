"""Drop-in EXL3 linear: ``ELinear`` / ``build_linear`` of runtime/ds41/exl3_linear.py:64-154,
forwarding to evamx_exl3_linear (fp16 in, fp16 out, the reference's rounding points).

Calls of up to 16 rows take the decode GEMV; larger calls take the MFMA path (the reference
likewise runs small batches row by row and hands larger ones to its GEMM, exl3_linear.py:106-128).
Within each path a row's result is independent of how many rows share the call (the k-split and
the per-row accumulation order depend only on in/out).

Strict dense mode (``DS41_STRICT_DENSE``, default on, exl3_linear.py:70,116-128): a call of up to
``verification_max_rows()`` rows runs as calls of at most 16 rows on the decode GEMV, so each row
keeps the bits it gets alone across every batch size up to that bound (the reference runs those
rows one at a time through its single-row kernel).
"""
from __future__ import annotations

import torch

from . import ops, verification

GEMV_MAX_ROWS = 16          # calls of up to this many rows take the decode GEMV (linear.hip)
MAX_CALL_ROWS = 65536       # rows per evamx_exl3_linear call


class ELinear:
    def __init__(self, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, *, strict: bool | None = None):
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
        self.strict_small_rows = verification.strict_dense() if strict is None else bool(strict)
        self._ws = None

    def _workspace(self, rows):
        need = ops.lib().evamx_exl3_linear_workspace_bytes(rows, self.in_features, self.out_features)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.trellis.device)
        return self._ws

    def call_rows(self, rows: int) -> int:
        """Rows per evamx_exl3_linear call for an input of ``rows`` rows."""
        if self.strict_small_rows and rows <= verification.verification_max_rows():
            return GEMV_MAX_ROWS
        return MAX_CALL_ROWS

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, shape[-1]).to(torch.float16).contiguous()
        if flat.shape[-1] != self.in_features:
            raise ValueError("input width differs from the EXL3 metadata")
        rows = flat.shape[0]
        y = torch.empty(rows, self.out_features, dtype=torch.float16, device=flat.device)
        step = self.call_rows(rows)
        for r0 in range(0, rows, step):
            part = flat[r0:r0 + step]
            ops.exl3_linear(part, self.trellis, self.suh, self.svh, self.k, out=y[r0:r0 + step],
                            workspace=self._workspace(part.shape[0]))
        return y.reshape(*shape[:-1], self.out_features)

    __call__ = forward


def build_linear(suh, svh, trellis, mul1=None, device: str = "cuda", *, strict: bool | None = None) -> ELinear:
    """exl3_linear.py:134-154. ``mul1`` only marks the MUL1 codebook, the only one supported."""
    suh = suh.to(device=device, dtype=torch.float16).contiguous()
    svh = svh.to(device=device, dtype=torch.float16).contiguous()
    trellis = trellis.to(device=device, dtype=torch.int16).contiguous()
    return ELinear(trellis, suh, svh, strict=strict)
