"""Tensor-level wrappers of the evamx C ABI (PyTorch-ROCm tensors in, device pointers out).

Every function launches HIP kernels from libevamx.so on the current stream; nothing here
computes on the CPU.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import MoeArgs, MoeShape, check, lib, ptr, stream_handle

SCORE_FNS = {"sigmoid": _lib.SCORE_SIGMOID, "sqrt_softplus": _lib.SCORE_SQRT_SOFTPLUS}
RATES = (2.0, 3.0, 4.0, 5.0)


def _dev(t: torch.Tensor, name: str, dtype=None, ndim=None, row_strided=False):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.ndim != ndim:
        raise ValueError(f"{name} must have {ndim} dims")
    if row_strided:
        if t.stride(-1) != 1 or (t.ndim == 2 and t.stride(0) < t.shape[1]):
            raise ValueError(f"{name} must have unit column stride and non-overlapping rows")
    elif not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def tile_u16(bits: float) -> int:
    b = float(bits)
    return 16 * int(b) + 8 if b != int(b) else 16 * int(b)


def exl3_dequant(trellis: torch.Tensor, bits: float) -> torch.Tensor:
    """fp16 ``W[in][out]`` of an EXL3 projection ``trellis int16 [in/16, out/16, T]``."""
    _dev(trellis, "trellis", torch.int16, 3)
    kt, nt, t16 = trellis.shape
    if t16 != tile_u16(bits):
        raise ValueError(f"trellis last dim {t16} does not match {bits} bits")
    w = torch.empty(kt * 16, nt * 16, dtype=torch.float16, device=trellis.device)
    check(lib().evamx_exl3_dequant(ptr(trellis), kt * 16, nt * 16, float(bits), ptr(w),
                                   stream_handle(trellis.device)), "evamx_exl3_dequant")
    return w


def exl3_linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, bits: float,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Single EXL3 linear, fp16 ``x [M, in]`` -> fp16 ``[M, out]`` (decode GEMV up to 16 rows, MFMA
    tiles beyond)."""
    _dev(x, "x", torch.float16, 2)
    _dev(trellis, "trellis", torch.int16, 3)
    _dev(suh, "suh", torch.float16, 1)
    _dev(svh, "svh", torch.float16, 1)
    m, n_in = x.shape
    n_out = svh.numel()
    if suh.numel() != n_in or trellis.shape[0] * 16 != n_in or trellis.shape[1] * 16 != n_out:
        raise ValueError("x / trellis / suh / svh shapes disagree")
    if out is None:
        out = torch.empty(m, n_out, dtype=torch.float16, device=x.device)
    _dev(out, "out", torch.float16, 2)
    if tuple(out.shape) != (m, n_out):
        raise ValueError(f"out must be [{m}, {n_out}]")
    need = lib().evamx_exl3_linear_workspace_bytes(m, n_in, n_out)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _dev(workspace, "workspace", torch.uint8, 1)
    check(lib().evamx_exl3_linear(ptr(x), m, n_in, n_out, ptr(trellis), ptr(suh), ptr(svh), float(bits), ptr(out),
                                  ptr(workspace), workspace.numel(), stream_handle(x.device)), "evamx_exl3_linear")
    return out


def route_topk(logits: torch.Tensor, topk: int, score_fn: str = "sigmoid", sel_bias: torch.Tensor | None = None,
               route_scale: float = 1.0):
    """(indices int64, weights fp32, rw fp16) of the top-k experts per row of ``logits [T, E]``."""
    _dev(logits, "logits", torch.float32, 2)
    t, e = logits.shape
    if sel_bias is not None:
        _dev(sel_bias, "sel_bias", torch.float32, 1)
    idx = torch.empty(t, topk, dtype=torch.int64, device=logits.device)
    w = torch.empty(t, topk, dtype=torch.float32, device=logits.device)
    rw = torch.empty(t, topk, dtype=torch.float16, device=logits.device)
    check(lib().evamx_route_topk(ptr(logits), ptr(sel_bias), t, e, topk, SCORE_FNS[score_fn], float(route_scale),
                                 ptr(idx), ptr(w), ptr(rw), stream_handle(logits.device)), "evamx_route_topk")
    return idx, w, rw


def router_logits(x: torch.Tensor, gate_w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``x.float() @ gate_w.T`` on the device (``evamx_router_logits``), each row reduced in one
    fixed order whatever the batch (model.py:158-165)."""
    if x.dim() != 2 or x.dtype not in (torch.float16, torch.bfloat16) or not x.is_cuda or x.stride(1) != 1:
        raise ValueError("x must be a CUDA fp16/bf16 [rows, hidden] tensor with unit inner stride")
    _dev(gate_w, "gate_w", torch.float32, 2)
    rows, hidden = x.shape
    if gate_w.shape[1] != hidden:
        raise ValueError(f"gate_w must be [n_experts, {hidden}]")
    if out is None:
        out = torch.empty(rows, gate_w.shape[0], dtype=torch.float32, device=x.device)
    _dev(out, "out", torch.float32, 2)
    check(lib().evamx_router_logits(ptr(x), _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F16, x.stride(0), rows,
                                    ptr(gate_w), gate_w.shape[0], hidden, ptr(out), stream_handle(x.device)),
          "evamx_router_logits")
    return out


def route(x: torch.Tensor, gate_w: torch.Tensor, gate_b: torch.Tensor | None, topk: int, route_scale: float = 1.0,
          score_fn: str = "sqrt_softplus", image_mask: torch.Tensor | None = None,
          gate_b_vl: torch.Tensor | None = None):
    """``Block.route(x, image_mask) -> (w, idx)`` (model.py:404-416) on the device: gate GEMV, scores,
    top-k of score + bias (``gate_b_vl`` for the rows of ``image_mask``), weights normalised and
    scaled. With a mask both biases are routed and the rows picked by ``torch.where`` (no host sync)."""
    z = router_logits(x, gate_w)
    idx, w, _ = route_topk(z, topk, score_fn, gate_b, route_scale)
    if image_mask is not None and gate_b_vl is not None:
        idx_vl, w_vl, _ = route_topk(z, topk, score_fn, gate_b_vl, route_scale)
        m = image_mask.reshape(-1, 1).to(device=z.device, dtype=torch.bool)
        idx = torch.where(m, idx_vl, idx)
        w = torch.where(m, w_vl, w)
    return w, idx


def prepare_routes_workspace_bytes(capacity: int, topk: int) -> int:
    n = lib().evamx_prepare_routes_workspace_bytes(capacity, topk)
    if n == 0:
        raise ValueError("invalid capacity/topk")
    return n


def prepare_routes(sel: torch.Tensor, rw: torch.Tensor, capacity: int, n_local: int,
                   runs: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The reference run table ``int32 [2 + 2*capacity*topk + 1]`` for routes ``sel``/``rw`` (fp16)."""
    _dev(sel, "sel", torch.int64, 2)
    _dev(rw, "rw", torch.float16, 2)
    t, k = sel.shape
    if rw.shape != sel.shape:
        raise ValueError("sel/rw shapes differ")
    if runs is None:
        runs = torch.empty(2 + 2 * capacity * k + 1, dtype=torch.int32, device=sel.device)
    need = lib().evamx_prepare_routes_workspace_bytes(capacity, k)
    if workspace is None:
        workspace = torch.zeros(need, dtype=torch.uint8, device=sel.device)
    check(lib().evamx_prepare_routes(ptr(sel), ptr(rw), t, k, capacity, n_local, ptr(runs), ptr(workspace),
                                     workspace.numel(), stream_handle(sel.device)), "evamx_prepare_routes")
    return runs


class MoeWorkspace:
    """Device workspace of the MoE forward for one shape (owned by one runner)."""

    def __init__(self, device, rows_max: int, hidden: int, inter: int, topk: int, n_local: int,
                 has_shared: bool, ksplit_gu: int = 0, ksplit_down: int = 0, strict_rows: int = 0):
        """``strict_rows`` > 0: calls of up to that many rows give every row the bits it gets in a
        one-row call (strict batch mode, the reference's DS41_STRICT_BATCH); 0: automatic geometry."""
        self.shape = MoeShape(rows_max, hidden, inter, topk, n_local, int(bool(has_shared)), ksplit_gu, ksplit_down,
                              strict_rows)
        nbytes = lib().evamx_moe_workspace_bytes(ctypes.byref(self.shape))
        if nbytes == 0:
            raise ValueError("invalid MoE shape: " + lib().evamx_last_error().decode())
        self.device = torch.device(device)
        self.buffer = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        check(lib().evamx_moe_workspace_init(ctypes.byref(self.shape), ptr(self.buffer), stream_handle(self.device)),
              "evamx_moe_workspace_init")

    def clear_flags(self) -> None:
        """Zero the sticky device flag word (a fill kernel on the current stream)."""
        check(lib().evamx_moe_workspace_init(ctypes.byref(self.shape), ptr(self.buffer), stream_handle(self.device)),
              "evamx_moe_workspace_init")

    def runs(self) -> torch.Tensor:
        """View of the run table written by the last forward."""
        slots = self.shape.rows_max * self.shape.topk
        addr = lib().evamx_moe_runs_ptr(ctypes.byref(self.shape), ptr(self.buffer))
        off = addr - self.buffer.data_ptr()
        n = 2 + 2 * slots + 1
        return self.buffer[off:off + 4 * n].view(torch.int32)

    def logits(self, rows: int, n_logits: int) -> torch.Tensor:
        """fp32 ``[rows, n_logits]`` router logits the last forward computed from ``gate_w``."""
        addr = lib().evamx_moe_logits_ptr(ctypes.byref(self.shape), ptr(self.buffer))
        off = addr - self.buffer.data_ptr()
        return self.buffer[off:off + 4 * rows * n_logits].view(torch.float32).view(rows, n_logits)

    def rotated(self) -> torch.Tensor:
        """fp16 ``[2, nslot_max, hidden]`` view of the rotated gate (0) and up (1) inputs the last
        forward of 3 or more rows wrote: routed slot ``row * topk + k``, shared-expert row ``r`` at
        ``rows * topk + r``."""
        s = self.shape
        nslot_max = s.rows_max * s.topk + (s.rows_max if s.has_shared else 0)
        addr = lib().evamx_moe_rotated_ptr(ctypes.byref(s), ptr(self.buffer))
        off = addr - self.buffer.data_ptr()
        n = 2 * nslot_max * s.hidden
        return self.buffer[off:off + 2 * n].view(torch.float16).view(2, nslot_max, s.hidden)

    def flags(self) -> torch.Tensor:
        addr = lib().evamx_moe_flags_ptr(ctypes.byref(self.shape), ptr(self.buffer))
        off = addr - self.buffer.data_ptr()
        return self.buffer[off:off + 4].view(torch.int32)


def _check_forward_args(s, device, x, tables, out, bits, k2_per_expert, logits, sel, weights, rw, sel_bias,
                        shared_ptrs, shared_bits, events, residual, gate_w):
    """Every tensor's device, dtype and shape against the workspace's shape, before any launch:
    the C ABI receives bare pointers and would read or write out of bounds otherwise."""
    def on_dev(t, name, dtype, shape=None, row_strided=False):
        _dev(t, name, dtype, len(shape) if shape is not None else None, row_strided=row_strided)
        if t.device != device:
            raise ValueError(f"{name} is on {t.device}, the workspace on {device}")
        if shape is not None:
            for i, (have, want) in enumerate(zip(t.shape, shape)):
                if want is not None and have != want:
                    raise ValueError(f"{name} must have shape {tuple('*' if w is None else w for w in shape)}, "
                                     f"got {tuple(t.shape)}")

    on_dev(x, "x", None, (None, s.hidden), row_strided=True)
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("x must be fp16 or bf16")
    rows, topk = x.shape[0], s.topk
    if not 1 <= rows <= s.rows_max:
        raise ValueError(f"x has {rows} rows, the workspace holds 1..{s.rows_max}")
    on_dev(tables, "tables", torch.int64, (9, s.n_local))
    if out is None and residual is None:
        raise ValueError("need out, residual or both")
    if out is not None:
        on_dev(out, "out", torch.float32, (None, None), row_strided=True)
        if out.shape[0] < rows or out.shape[1] < s.hidden:
            raise ValueError(f"out must be at least [{rows}, {s.hidden}], got {tuple(out.shape)}")
    if residual is not None:
        on_dev(residual, "residual", torch.bfloat16, (rows, None), row_strided=True)
        if residual.shape[1] < s.hidden:
            raise ValueError(f"residual must be [{rows}, >= {s.hidden}]")
    if sel is None:
        raise ValueError("sel is required (routes in, or the routing's output)")
    on_dev(sel, "sel", torch.int64, (rows, topk))
    if weights is not None:
        on_dev(weights, "weights", torch.float32, (rows, topk))
    if rw is not None:
        on_dev(rw, "rw", torch.float16, (rows, topk))
    if logits is not None and gate_w is not None:
        raise ValueError("give logits or gate_w, not both")
    routing = logits is not None or gate_w is not None
    if routing:
        if weights is None:
            raise ValueError("routing on the device writes weights: pass an fp32 [rows, topk] output")
        if logits is not None:
            on_dev(logits, "logits", torch.float32, (rows, None))
            n_logits = logits.shape[1]
        else:
            on_dev(gate_w, "gate_w", torch.float32, (None, s.hidden))
            n_logits = gate_w.shape[0]
        if not topk <= n_logits <= 512:
            raise ValueError(f"{n_logits} experts in the router, need {topk}..512")
        if sel_bias is not None:
            on_dev(sel_bias, "sel_bias", torch.float32, (n_logits,))
    elif weights is None and rw is None:
        raise ValueError("given routes need fp32 weights or fp16 rw")
    elif sel_bias is not None:
        raise ValueError("sel_bias applies only when routing on the device")
    if k2_per_expert is not None:
        on_dev(k2_per_expert, "k2_per_expert", torch.uint8, (s.n_local,))
    elif bits is None:
        raise ValueError("give a uniform rate (bits) or k2_per_expert")
    if s.has_shared:
        if shared_ptrs is None or len(shared_ptrs) != 9 or shared_bits is None:
            raise ValueError("the workspace has a shared expert: pass its 9 pointers and shared_bits")
    elif shared_ptrs is not None:
        raise ValueError("the workspace was built without a shared expert")
    if events is not None and len(events) != 10:
        raise ValueError("events must hold 10 event handles")


def _moe_args(s, device, x, tables, out, limit, bits, k2_per_expert, logits, sel, weights, rw, score_fn, sel_bias,
              route_scale, shared_ptrs, shared_bits, min_expert, max_expert, events, residual, gate_w,
              bits_down=None, k2_down_per_expert=None, shared_bits_down=None, shared_gate_w=None):
    """The evamx_moe_args of one forward call (every tensor checked first), without the
    workspace; returns it with the ctypes array of shared pointers it refers to."""
    _check_forward_args(s, device, x, tables, out, bits, k2_per_expert, logits, sel, weights, rw, sel_bias,
                        shared_ptrs, shared_bits, events, residual, gate_w)
    if k2_down_per_expert is not None:
        _dev(k2_down_per_expert, "k2_down_per_expert", torch.uint8, 1)
        if k2_down_per_expert.device != device or k2_down_per_expert.numel() != s.n_local:
            raise ValueError(f"k2_down_per_expert must be a uint8 [{s.n_local}] tensor on {device}")
    if shared_gate_w is not None:
        _dev(shared_gate_w, "shared_gate_w", torch.float16, 1)
        if shared_gate_w.device != device or shared_gate_w.numel() != s.hidden:
            raise ValueError(f"shared_gate_w must be an fp16 [{s.hidden}] tensor on {device}")
        if not s.has_shared:
            raise ValueError("shared_gate_w needs a shared expert")
    a = MoeArgs()
    a.shape = s
    a.rows = x.shape[0]
    a.x = ptr(x)
    a.x_dtype = _lib.DTYPE_F16 if x.dtype == torch.float16 else _lib.DTYPE_BF16
    a.x_stride = x.stride(0)
    if logits is not None or gate_w is not None:
        if logits is not None:
            a.logits = ptr(logits)
            a.n_logits = logits.shape[1]
        else:
            a.gate_w = ptr(gate_w)
            a.n_logits = gate_w.shape[0]
        a.sel_bias = ptr(sel_bias)
        a.score_fn = SCORE_FNS[score_fn]
        a.route_scale = float(route_scale)
    a.sel = ptr(sel)
    a.weights = ptr(weights)
    a.rw_fp16 = ptr(rw)
    a.min_expert = min_expert
    a.max_expert = max_expert
    a.tables = ptr(tables)
    a.k2_per_expert = ptr(k2_per_expert)
    a.bits = float(bits) if bits is not None else 0.0
    keep = None
    if shared_ptrs is not None:
        keep = (ctypes.c_int64 * 9)(*[int(v) for v in shared_ptrs])
        a.shared = ctypes.cast(keep, ctypes.c_void_p)
        a.shared_bits = float(shared_bits)
    a.limit = float(limit)
    a.out = ptr(out)
    a.out_stride = out.stride(0) if out is not None else 0
    if residual is not None:
        a.residual = ptr(residual)
        a.residual_stride = residual.stride(0)
    if events is not None:
        a.events = ctypes.cast(events, ctypes.c_void_p)
    a.bits_down = float(bits_down) if bits_down is not None else 0.0
    a.k2_down_per_expert = ptr(k2_down_per_expert)
    a.shared_bits_down = float(shared_bits_down) if shared_bits_down is not None else 0.0
    a.shared_gate_w = ptr(shared_gate_w)
    return a, keep


def moe_forward(ws: MoeWorkspace, x: torch.Tensor, tables: torch.Tensor, out: torch.Tensor | None, *, limit: float,
                bits: float | None = None, k2_per_expert: torch.Tensor | None = None,
                logits: torch.Tensor | None = None, sel: torch.Tensor | None = None,
                weights: torch.Tensor | None = None, rw: torch.Tensor | None = None,
                score_fn: str = "sigmoid", sel_bias: torch.Tensor | None = None, route_scale: float = 1.0,
                shared_ptrs=None, shared_bits: float | None = None, min_expert: int = -1, max_expert: int = 0,
                events=None, residual: torch.Tensor | None = None, gate_w: torch.Tensor | None = None,
                bits_down: float | None = None, k2_down_per_expert: torch.Tensor | None = None,
                shared_bits_down: float | None = None, shared_gate_w: torch.Tensor | None = None):
    """One MoE layer: out[r] = sum over r's active slots (slot order) + shared expert.

    With ``logits`` the routing runs on the device and writes ``sel``/``weights``/``rw`` (all
    must be given as outputs); otherwise ``sel`` with ``weights`` (fp32) or ``rw`` (fp16) are
    the routes. ``tables``: int64 ``[9, n_local]`` device pointer table. ``shared_ptrs``: 9 ints.
    ``events``: optional ctypes array of 10 hipEvent_t handles: start and end timestamps of the
    5 stages' kernels (prepare, gate/up, activation, down, combine).
    ``residual``: optional bf16 ``[rows, H]`` stream updated in place to ``bf16(residual + bf16(y))``
    (may be ``x`` itself); ``out`` may then be None.
    ``gate_w``: optional fp32 ``[n_experts, H]`` router weight; the logits ``x @ gate_w.T`` are then
    computed on the device (instead of ``logits``) and routed with ``score_fn``/``sel_bias``.
    ``bits_down`` / ``k2_down_per_expert`` / ``shared_bits_down``: the down projections' rate when
    it differs from gate/up (the reference launcher's K_d). ``shared_gate_w``: fp16 ``[H]``; the
    shared term is then scaled by sigmoid(x . shared_gate_w) per row.
    """
    a, keep = _moe_args(ws.shape, ws.buffer.device, x, tables, out, limit, bits, k2_per_expert, logits, sel, weights,
                        rw, score_fn, sel_bias, route_scale, shared_ptrs, shared_bits, min_expert, max_expert, events,
                        residual, gate_w, bits_down, k2_down_per_expert, shared_bits_down, shared_gate_w)
    a.workspace = ptr(ws.buffer)
    a.workspace_bytes = ws.buffer.numel()
    check(lib().evamx_moe_forward(ctypes.byref(a), stream_handle(x.device)), "evamx_moe_forward")
    del keep
    return out


def moe_forward_static(shape: MoeShape, x: torch.Tensor, tables: torch.Tensor, out: torch.Tensor | None, *,
                       limit: float, bits: float | None = None, k2_per_expert: torch.Tensor | None = None,
                       logits: torch.Tensor | None = None, sel: torch.Tensor | None = None,
                       weights: torch.Tensor | None = None, rw: torch.Tensor | None = None,
                       score_fn: str = "sigmoid", sel_bias: torch.Tensor | None = None, route_scale: float = 1.0,
                       shared_ptrs=None, shared_bits: float | None = None, min_expert: int = -1,
                       max_expert: int = 0, events=None, residual: torch.Tensor | None = None,
                       gate_w: torch.Tensor | None = None, bits_down: float | None = None,
                       k2_down_per_expert: torch.Tensor | None = None, shared_bits_down: float | None = None,
                       shared_gate_w: torch.Tensor | None = None):
    """``moe_forward`` without a workspace: evamx_moe_forward_static runs the layer on the
    library's fixed device scratch (64 MiB per GPU) and allocates nothing, for callers that
    cannot allocate (e.g. under graph capture). ``shape`` is the MoeShape a workspace would have
    been built for. Calls that overlap on one GPU share the scratch and race."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        raise ValueError("x must be a device tensor")
    a, keep = _moe_args(shape, x.device, x, tables, out, limit, bits, k2_per_expert, logits, sel, weights, rw,
                        score_fn, sel_bias, route_scale, shared_ptrs, shared_bits, min_expert, max_expert, events,
                        residual, gate_w, bits_down, k2_down_per_expert, shared_bits_down, shared_gate_w)
    check(lib().evamx_moe_forward_static(ctypes.byref(a), stream_handle(x.device)), "evamx_moe_forward_static")
    del keep
    return out


def read_floor(ncg: int, rows: int, waves: int, device=None, reps: int = 50) -> float:
    """Bytes per second of the read-only benchmark (evamx_bench_read): ``waves`` waves stream
    ``rows`` 1 KiB chunks each in a decode GEMV launch's shape (wave w reads column group w % ncg
    of its chain's rows), no decode; ``reps`` back-to-back launches timed with events. The
    launches cycle through distinct copies totalling at least 1 GiB, as the layer benchmark
    cycles its weights, so that the 256 MiB Infinity Cache cannot serve a repeated buffer."""
    dev = torch.device("cuda", 0) if device is None else torch.device(device)
    nbytes = (waves // ncg) * rows * ncg * 1024
    copies = min(64, max(2, -(-(1 << 30) // nbytes)))
    buf = torch.zeros(copies * nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(64, dtype=torch.float32, device=dev)
    stream = stream_handle(dev)
    base = ptr(buf)

    def launch(i):
        check(lib().evamx_bench_read(base + (i % copies) * nbytes, nbytes, ncg, rows, waves, ptr(sink), stream),
              "evamx_bench_read")

    for i in range(copies):   # warm-up: every copy once
        launch(i)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        launch(i)
    e1.record()
    e1.synchronize()
    return nbytes * reps / (e0.elapsed_time(e1) * 1e-3)


def decode_ceiling(bits: float, device=None, waves: int | None = None, iters: int = 4000) -> float:
    """Decoded weights per second of the register-only decode benchmark (evamx_bench_decode):
    the arithmetic bound of the decode GEMV at ``bits``, timed with events on the current stream."""
    dev = torch.device("cuda", 0) if device is None else torch.device(device)
    if waves is None:
        waves = torch.cuda.get_device_properties(dev).multi_processor_count * 16
    sink = torch.zeros(256, dtype=torch.float32, device=dev)
    stream = stream_handle(dev)
    check(lib().evamx_bench_decode(float(bits), waves, 16, ptr(sink), stream), "evamx_bench_decode")   # warm-up
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    check(lib().evamx_bench_decode(float(bits), waves, iters, ptr(sink), stream), "evamx_bench_decode")
    e1.record()
    e1.synchronize()
    return waves * 64.0 * 32.0 * iters / (e0.elapsed_time(e1) * 1e-3)
