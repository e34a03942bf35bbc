"""Helpers shared by the GPU parity tests: upload oracle-side synthetic experts to the device and
build the ``[9, n_local]`` pointer table the kernels read (reference layout, cache.py:1877-1886)."""
from __future__ import annotations

import numpy as np
import torch


def to_dev(a, device, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(device)


class DeviceExperts:
    """Device copies of a list of oracle ExpertWeights plus their pointer table."""

    def __init__(self, experts, device):
        self.keep = []
        self.rows = []
        for ew in experts:
            ptrs = []
            for p in ("g", "u", "d"):
                tr, suh, svh = ew.parts[p]
                t_tr = to_dev(tr, device)
                t_suh = to_dev(suh, device)
                t_svh = to_dev(svh, device)
                self.keep += [t_tr, t_suh, t_svh]
                ptrs += [t_tr.data_ptr(), t_suh.data_ptr(), t_svh.data_ptr()]
            self.rows.append(ptrs)
        table = np.array(self.rows, dtype=np.int64).T.copy()     # [9, n]
        self.table = torch.from_numpy(table).to(device)
        self.k2 = torch.tensor([int(round(2 * ew.K)) for ew in experts], dtype=torch.uint8, device=device)
        self.k2_down = torch.tensor([int(round(2 * ew.K_down)) for ew in experts], dtype=torch.uint8, device=device)

    def ptrs(self, i):
        return self.rows[i]


def rel_err_rows(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float((np.abs(y - ref).max(axis=-1) / np.maximum(np.abs(ref).max(axis=-1), 1e-30)).max())


def clamp_variants(compute):
    """``compute()`` under the oracle's activation semantics and three wrong ones, to give a
    test of the SwiGLU limit teeth: the reference clamps a routed expert's gate AFTER SiLU
    (exl3_moe_coop_kernel.cuh:115-129) and the shared expert's gate BEFORE SiLU
    (kernels.py:213-217). Returns {"ref", "routed_swapped", "shared_swapped", "unclamped"}."""
    from oracle import coop

    act, sw = coop.act_gate, coop.swiglu
    out = {"ref": compute()}
    variants = {"routed_swapped": (lambda g, u, L: sw(g, u, L), sw),
                "shared_swapped": (act, lambda g, u, L: act(g, u, L)),
                "unclamped": (lambda g, u, L: act(g, u, 0.0), lambda g, u, L: sw(g, u, 0.0))}
    try:
        for name, (a, s) in variants.items():
            coop.act_gate, coop.swiglu = a, s
            out[name] = compute()
    finally:
        coop.act_gate, coop.swiglu = act, sw
    return out
