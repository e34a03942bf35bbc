"""Strict batch mode and the runner-side names on the host (no GPU): the verification bound's
accepted spellings (runtime/ds41/verification.py:15-30), the strict row count a MoE workspace gets
(DS41_STRICT_BATCH, moe_coop.py:17-22), ``WorkspaceLayout`` / ``source_metadata`` as the production
owner imports them (native3072_runtime.py:134,146; moe_coop3072.py:120-152), and how ``ELinear``
cuts a call into library calls (0 rows, above 65536 rows, strict dense mode)."""
import ctypes

import numpy as np
import pytest
import torch

from eva_amd import _lib, coop, linear, ops, verification


@pytest.mark.parametrize("v,ok", [("8", 8), ("1", 1), ("128", 128), ("256", 256), ("512", 512), ("1024", 1024),
                                  (" 64", 64), ("0", None), ("129", None), ("300", None), ("2048", None),
                                  ("08", None), ("8.0", None), ("x", None), (8, None)])
def test_verification_bound_spellings(v, ok):
    if ok is None:
        with pytest.raises(ValueError):
            verification.parse_max_rows(v)
    else:
        assert verification.parse_max_rows(v) == ok


def test_moe_strict_rows(monkeypatch):
    assert verification.moe_strict_rows(512, 6, strict=True, bound=8) == 8
    assert verification.moe_strict_rows(4, 8, strict=True, bound=8) == 4           # capped by the capacity
    assert verification.moe_strict_rows(512, 6, strict=False, bound=8) == 0
    assert verification.moe_strict_rows(16, 8, strict=True, bound=16) == 16
    with pytest.raises(ValueError):
        verification.moe_strict_rows(512, 8, strict=True, bound=64)                 # 512 slots > 256
    with pytest.raises(ValueError):
        verification.moe_strict_rows(512, 1, strict=True, bound=128)                # rows > 64
    monkeypatch.setenv("DS41_STRICT_BATCH", "0")
    assert verification.moe_strict_rows(512, 6) == 0
    monkeypatch.setenv("DS41_STRICT_BATCH", "1")
    assert verification.moe_strict_rows(512, 6) == min(512, verification.verification_max_rows())


def test_workspace_layout_matches_the_c_abi():
    L = coop.WorkspaceLayout()                       # the reference's defaults: 512 x H5120/I2304, top-6
    assert (L.max_rows, L.hidden, L.inter, L.topk, L.slots) == (512, 5120, 2304, 6, 3072)
    assert L.run_table_ints == 2 + 2 * 3072 + 1
    for strict in (0, 8):
        L = coop.WorkspaceLayout(max_rows=16, hidden=7168, inter=2048, topk=8, n_local=256, has_shared=True,
                                 strict_rows=strict)
        shape = _lib.MoeShape(16, 7168, 2048, 8, 256, 1, 0, 0, strict)
        ws = _lib.lib().evamx_moe_workspace_bytes(ctypes.byref(shape))
        assert L.moe_workspace_bytes == ws > 0
        assert L.scratch_bytes == (ws + 16 * 7168 * 4 + 16 * 8 * 2 + (2 + 2 * 128 + 1) * 4
                                   + ops.prepare_routes_workspace_bytes(16, 8))
    with pytest.raises(ValueError):
        coop.WorkspaceLayout(hidden=5000)
    with pytest.raises(ValueError):
        coop.WorkspaceLayout(max_rows=0)


def test_source_metadata_identity():
    from eva_amd import build
    m = coop.source_metadata()
    assert m["abi_version"] == _lib.ABI_VERSION == _lib.lib().evamx_abi_version()
    assert m["arch"] == "gfx950" and m["hipcc_flags"] == list(build.FLAGS)
    assert len(m["source_sha256"]) == 64 and len(m["build_sha256"]) == 64
    assert m["source_files"] >= len(build.sources())
    assert m == coop.source_metadata()                # deterministic
    # the names the production owner imports next to the runner class
    from eva_amd.coop import CoopRunner3072, WorkspaceLayout, source_metadata  # noqa: F401


class _Recorder:
    def __init__(self):
        self.rows = []

    def __call__(self, x, trellis, suh, svh, bits, out=None, workspace=None):
        assert x.is_contiguous() and out.is_contiguous() and out.shape[0] == x.shape[0]
        self.rows.append(x.shape[0])
        out.fill_(1.0)
        return out


@pytest.fixture
def cpu_linear(monkeypatch):
    rec = _Recorder()
    monkeypatch.setattr(ops, "exl3_linear", rec)
    monkeypatch.setattr(linear.ELinear, "_workspace", lambda self, rows: None)
    tr = torch.zeros(128 // 16, 256 // 16, 64, dtype=torch.int16)
    make = lambda strict: linear.ELinear(tr, torch.ones(128, dtype=torch.float16), torch.ones(256, dtype=torch.float16),
                                         strict=strict)
    return make, rec


def test_elinear_call_splitting(cpu_linear):
    make, rec = cpu_linear
    lin = make(False)
    y = lin.forward(torch.zeros(0, 128))
    assert tuple(y.shape) == (0, 256) and rec.rows == []        # 0 rows: no library call
    y = lin.forward(torch.zeros(3, 0, 128))
    assert tuple(y.shape) == (3, 0, 256)
    rec.rows.clear()
    y = lin.forward(torch.zeros(70000, 128))                  # above the C ABI's 65536 rows per call
    assert rec.rows == [65536, 70000 - 65536] and bool((y == 1).all())
    rec.rows.clear()
    lin.forward(torch.zeros(100, 128))
    assert rec.rows == [100]


def test_elinear_strict_dense_keeps_the_gemv(cpu_linear):
    make, rec = cpu_linear
    lin = make(True)
    bound = verification.verification_max_rows()
    for rows in sorted({1, 2, 16, bound, bound + 1, 100}):
        rec.rows.clear()
        lin.forward(torch.zeros(rows, 128))
        if rows <= bound:
            assert max(rec.rows) <= linear.GEMV_MAX_ROWS and sum(rec.rows) == rows
        else:
            assert rec.rows == [rows]
    assert make(None).strict_small_rows == verification.strict_dense()
