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

    def ptrs(self, i):
        return self.rows[i]


def rel_err_rows(y, ref):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float((np.abs(y - ref).max(axis=-1) / np.maximum(np.abs(ref).max(axis=-1), 1e-30)).max())
