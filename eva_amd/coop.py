"""Drop-in runners for eva's cooperative EXL3 MoE operator, on libevamx.

Mirrors the reference's Python interface so callers switch by import:

- ``CoopRunner(device, topk, hidden, inter, rows=1).run(x, sel, weights, packed, k, limit)``
  -> borrowed fp32 ``[rows, hidden]`` (runtime/ds41/moe_coop.py:15-69);
- ``CoopRunner512/2048/3072(device, topk=6, hidden=5120, inter=2304, max_rows=...)`` with
  ``run(..., check_bounds=True)`` -> fp32 ``[M, hidden]``, ``prepare_routes``,
  ``run_table``, ``lifecycle``, ``close`` (runtime/ds41/moe_coop3072.py:261-402,
  moe_coop512.py:170-253, moe_coop2048.py:220-351), with their ownership rules: one owner
  thread, the construction stream, a non-blocking lock, and any failure poisons the runner.
  CoopRunner512 returns the runner's own output rows (borrowed), as moe_coop512.py:248 does.

Generalised as the DeepSeek-V3 shapes need: any hidden/inter (multiples of 128), top-k up to
32, up to 512 local experts, rates 1.5 to 4 bits in steps of 0.5 and 5 bits. ``packed`` is the ``[9, n_local]`` int64
pointer table (rows g_trellis, g_suh, g_svh, u_trellis, u_suh, u_svh, d_trellis, d_suh,
d_svh; runtime/ds41/cache.py:1877-1886) or a sequence of its 9 rows.

Differences, all on the side of fewer host round trips:

- bounds: the reference checks expert indices with a host synchronisation before launching
  (csrc/moe_coop3072/moe_coop3072.cu:121-124). Here the kernels flag out-of-range experts in
  the workspace and skip those slots; ``check_bounds=True`` reads the flag after the launch
  (one synchronisation, as in the reference) and raises, poisoning the runner.
  ``check_bounds=False`` skips the read and allows graph capture.
- the run table is rebuilt by every ``run`` (as in the reference) and is the same int32 layout.
"""
from __future__ import annotations

import contextlib
import ctypes
import dataclasses
import hashlib
import json
import math
import os
import threading

import torch

from . import ops
from . import verification

RATES = (1.5, 2, 2.5, 3, 3.5, 4, 5)


def _pointer_table(packed, device, n_local=None):
    """``[9, n]`` int64 device table from a tensor or a sequence of 9 row tensors."""
    if isinstance(packed, torch.Tensor):
        t = packed
    elif isinstance(packed, (tuple, list)) and len(packed) == 9:
        rows = list(packed)
        if any(not isinstance(r, torch.Tensor) or r.ndim != 1 for r in rows):
            raise ValueError("pointer table rows must be 1-D tensors")
        base = rows[0]
        n = base.numel()
        contiguous_view = all(r.dtype == torch.int64 and r.numel() == n and r.stride(0) == 1
                              and r.data_ptr() == base.data_ptr() + 8 * n * i for i, r in enumerate(rows))
        t = (torch.as_strided(base, (9, n), (n, 1)) if contiguous_view else torch.stack(rows))
    else:
        raise ValueError("packed must be a [9, n_local] tensor or nine row tensors")
    if t.ndim != 2 or t.shape[0] != 9 or t.dtype != torch.int64 or t.device != device:
        raise ValueError("pointer table must be int64 [9, n_local] on the runner device")
    if n_local is not None and t.shape[1] != n_local:
        raise ValueError(f"pointer table has {t.shape[1]} experts, runner expects {n_local}")
    return t.contiguous()


def _check_rate(k):
    if type(k) not in (int, float) or float(k) not in RATES:
        raise ValueError(f"supported uniform rates are {RATES} bits")
    return float(k)


def _check_limit(limit):
    if type(limit) not in (int, float) or not math.isfinite(limit) or not 0 <= limit <= 3.4028234663852886e38:
        raise ValueError("limit must be a finite nonnegative float")
    return float(limit)


class CoopRunner:
    """Fixed-row decode runner (runtime/ds41/moe_coop.py:15-69). ``run`` returns a borrowed
    fp32 ``[rows, hidden]`` that the next call overwrites."""

    def __init__(self, device, topk: int, hidden: int, inter: int, rows: int = 1, n_local: int | None = None,
                 *, strict_rows: int | None = None):
        slots = topk * rows
        if rows < 1 or slots > 256:
            raise ValueError("Cooperative EXL3 supports 1..256 routed slots")
        # strict batch mode (DS41_STRICT_BATCH, default on; moe_coop.py:17-22): calls of up to the
        # verification bound compute every row as a one-row call would
        self.strict_rows = verification.moe_strict_rows(rows, topk) if strict_rows is None else strict_rows
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("CoopRunner needs a GPU device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.topk, self.rows, self.hi, self.inter, self.ho = topk, rows, hidden, inter, hidden
        self.n_local = n_local
        self._ws = {}
        self.out = torch.empty(rows, hidden, device=self.device, dtype=torch.float32)
        self.rw = torch.empty(rows, topk, device=self.device, dtype=torch.float16)

    def _workspace(self, n_local):
        ws = self._ws.get(n_local)
        if ws is None:
            ws = ops.MoeWorkspace(self.device, rows_max=self.rows, hidden=self.hi, inter=self.inter, topk=self.topk,
                                  n_local=n_local, has_shared=False, strict_rows=self.strict_rows)
            self._ws[n_local] = ws
        return ws

    def run(self, x, sel, weights, packed, k, limit) -> torch.Tensor:
        table = _pointer_table(packed, self.device, self.n_local)
        ws = self._workspace(table.shape[1])
        x = x.reshape(self.rows, self.hi).contiguous()
        if x.dtype not in (torch.float16, torch.bfloat16):
            x = x.to(torch.float16)
        sel = sel.reshape(self.rows, self.topk).to(dtype=torch.long).contiguous()
        self.rw.copy_(weights.reshape(self.rows, self.topk).to(dtype=torch.float16))
        ops.moe_forward(ws, x, table, self.out, limit=_check_limit(limit), bits=_check_rate(k), sel=sel, rw=self.rw)
        return self.out


class _Ownership:
    """The reference runners' usage contract (moe_coop3072.py:261-402) as one guard: calls come
    from the thread that built the runner, on the stream that was current then, one at a time
    (a second concurrent call is refused, not queued); an exception inside a guarded call
    poisons the runner for good; once closed it accepts nothing. ``leases`` keeps the tensors a
    failed call had handed to the GPU alive until a successful close has drained the stream."""

    def __init__(self, device):
        self.device = device
        self.stream = torch.cuda.current_stream(device)
        self.tid = threading.get_ident()
        self.busy = threading.Lock()
        self.poisoned = False
        self.shut = False
        self.drains = 0
        self.leases = []

    def on_owner_thread(self):
        return threading.get_ident() == self.tid

    @contextlib.contextmanager
    def call(self, what, capture_ok=False):
        if not self.on_owner_thread():
            raise RuntimeError(f"{what}: only the thread that built this runner may call it")
        if self.poisoned or self.shut:
            raise RuntimeError(f"{what}: this runner is {'poisoned by an earlier failure' if self.poisoned else 'closed'}"
                               "; build a new one")
        if torch.cuda.current_stream(self.device).cuda_stream != self.stream.cuda_stream:
            raise RuntimeError(f"{what}: call on the stream the runner was built on (streams are never switched "
                               "implicitly)")
        if not capture_ok:
            with torch.cuda.device(self.device):
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError(f"{what}: not capturable, it reads a device value back to the host")
        if not self.busy.acquire(blocking=False):
            raise RuntimeError(f"{what}: the runner is busy with another call")
        try:
            yield
        except BaseException:
            self.poisoned = True
            raise
        finally:
            self.busy.release()

    def lease(self, tensors):
        """Tie ``tensors`` to the runner's stream (record_stream) and hold them until the call
        that launched work on them has returned."""
        self.leases = list(tensors)
        for t in self.leases:
            t.record_stream(self.stream)

    def release(self):
        self.leases = []

    def close(self):
        if not self.on_owner_thread():
            raise RuntimeError("close: only the thread that built this runner may close it")
        if self.shut:
            return
        if not self.busy.acquire(blocking=False):
            raise RuntimeError("close: the runner is busy with another call")
        try:
            try:
                self.stream.synchronize()
            except BaseException:
                self.poisoned = True          # the leases stay held: the GPU may still use them
                raise
            self.drains += 1
            self.leases = []
            self.shut = True
        finally:
            self.busy.release()

    def state(self):
        # keys are the reference's lifecycle() report, which callers read
        return {"failed": self.poisoned, "closed": self.shut, "close_drains": self.drains,
                "owner_thread_matches": self.on_owner_thread(), "failed_input_leases": len(self.leases),
                "workspace_owners_retained": True, "caller_weight_pointer_lease_required": True,
                "raw_addresses_disclosed": False}


class CoopRunnerCapacity:
    """Bounded-capacity runner with the ownership rules of CoopRunner3072
    (runtime/ds41/moe_coop3072.py:261-402). Subclasses fix the default capacity and whether
    ``run`` hands back the runner's own output rows (borrowed) or a copy (owned)."""

    DEFAULT_MAX_ROWS = 512
    OWNED_OUTPUT = True

    def __init__(self, device="cuda", topk=6, hidden=5120, inter=2304, max_rows=None, *, n_local=None,
                 verbose=False, strict_rows=None):
        max_rows = self.DEFAULT_MAX_ROWS if max_rows is None else max_rows
        if type(topk) is not int or not 1 <= topk <= 32:
            raise ValueError("topk must be an integer in 1..32")
        if type(max_rows) is not int or not 1 <= max_rows <= 65536 // topk:
            raise ValueError("max_rows out of range")
        if hidden % 128 or inter % 128 or hidden < 128 or inter < 128:
            raise ValueError("hidden and inter must be positive multiples of 128")
        if not torch.cuda.is_available():
            raise RuntimeError("the MoE runner requires a GPU; there is no CPU numerical fallback")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the MoE runner requires a GPU device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        with torch.cuda.device(self.device):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("runner construction during capture is unsupported")
        self.topk, self.hidden, self.inter, self.max_rows = topk, hidden, inter, max_rows
        self.n_local = n_local
        # strict batch mode (DS41_STRICT_BATCH, default on: moe_coop.py:17-22, cache.py:2088-2091):
        # calls of up to the verification bound give every row the bits of a one-row call
        self.strict_rows = verification.moe_strict_rows(max_rows, topk) if strict_rows is None else strict_rows
        self.verbose = verbose
        self._own = _Ownership(self.device)
        self._table_valid = False
        self._ws = {}
        self._last_ws = None
        self.out = torch.empty(max_rows, hidden, device=self.device, dtype=torch.float32)
        self.rw = torch.empty(max_rows, topk, device=self.device, dtype=torch.float16)
        self.table = torch.zeros(2 + 2 * max_rows * topk + 1, device=self.device, dtype=torch.int32)
        self._prep_ws = torch.zeros(ops.prepare_routes_workspace_bytes(max_rows, topk), device=self.device,
                                    dtype=torch.uint8)

    # -- helpers -------------------------------------------------------------------------------

    def _workspace(self, n_local):
        ws = self._ws.get(n_local)
        if ws is None:
            ws = ops.MoeWorkspace(self.device, rows_max=self.max_rows, hidden=self.hidden, inter=self.inter,
                                  topk=self.topk, n_local=n_local, has_shared=False, strict_rows=self.strict_rows)
            self._ws[n_local] = ws
        return ws

    def _check_routes(self, sel, weights, rows):
        """sel: int64 [rows, topk]; weights: fp16/bf16/fp32 of the same shape; both on the
        runner's device."""
        if not isinstance(sel, torch.Tensor) or sel.dtype != torch.int64 or tuple(sel.shape) != (rows, self.topk):
            raise ValueError(f"sel: expected an int64 tensor of shape ({rows}, {self.topk})")
        if (not isinstance(weights, torch.Tensor) or weights.shape != sel.shape
                or weights.dtype not in (torch.float16, torch.bfloat16, torch.float32)):
            raise ValueError(f"weights: expected a floating tensor (fp16, bf16 or fp32) of shape ({rows}, {self.topk})")
        if sel.device != self.device or weights.device != self.device:
            raise ValueError(f"sel and weights must live on {self.device}")

    def _check_x(self, x):
        if (not isinstance(x, torch.Tensor) or x.ndim != 2 or x.shape[1] != self.hidden
                or not 1 <= x.shape[0] <= self.max_rows or x.dtype not in (torch.float16, torch.bfloat16)):
            raise ValueError(f"x: expected an fp16 or bf16 tensor of shape (1..{self.max_rows}, {self.hidden})")
        if x.device != self.device:
            raise ValueError(f"x must live on {self.device}")
        return x.shape[0]

    # -- reference API ---------------------------------------------------------------------------

    def run(self, x, sel, weights, packed, k, limit, *, check_bounds=True):
        """Run M rows; fp32 ``[M, hidden]``, owned or borrowed (``OWNED_OUTPUT``). Pointer
        targets are leased by the caller until the GPU is done with them."""
        k = _check_rate(k)
        limit = _check_limit(limit)
        if check_bounds not in (True, False):
            raise ValueError("check_bounds must be a bool")
        rows = self._check_x(x)
        self._check_routes(sel, weights, rows)
        table = _pointer_table(packed, self.device, self.n_local)
        with self._own.call("run", capture_ok=not check_bounds):
            x, sel = x.contiguous(), sel.contiguous()
            ws = self._workspace(table.shape[1])
            self._own.lease([x, sel, weights, table, ws.buffer, self.out, self.rw])
            rw = self.rw[:rows]
            rw.copy_(weights.to(torch.float16))
            ws.clear_flags()
            out = self.out[:rows]
            ops.moe_forward(ws, x, table, out, limit=limit, bits=k, sel=sel, rw=rw)
            self._last_ws = ws
            self._table_valid = True
            if check_bounds and int(ws.flags()[0].item()) != 0:
                raise RuntimeError("expert index outside the pointer table")
            result = out.clone() if self.OWNED_OUTPUT else out
            self._own.release()
            return result

    def prepare_routes(self, sel, weights, n_local):
        """The run table of these routes (owned int32 ``[2 + 2*max_rows*topk + 1]``)."""
        if type(n_local) is not int or not 1 <= n_local <= 512:
            raise ValueError("n_local must be an integer in 1..512")
        if not isinstance(sel, torch.Tensor) or sel.ndim != 2 or not 1 <= sel.shape[0] <= self.max_rows:
            raise ValueError(f"sel: expected a 2-D tensor of 1..{self.max_rows} rows")
        self._check_routes(sel, weights, sel.shape[0])
        with self._own.call("prepare_routes"):
            sel = sel.contiguous()
            self._own.lease([sel, weights, self.rw, self.table, self._prep_ws])
            rw = self.rw[:len(sel)]
            rw.copy_(weights.to(torch.float16))
            self._prep_ws[:4].zero_()
            ops.prepare_routes(sel, rw, self.max_rows, n_local, runs=self.table, workspace=self._prep_ws)
            self._last_ws = None
            self._table_valid = True
            result = self.table.clone()
            self._own.release()
            return result

    def run_table(self):
        """Owned snapshot of the last run's (or prepare's) table."""
        if not self._table_valid:
            raise RuntimeError("run_table: no run or prepare_routes has filled a table yet")
        with self._own.call("run_table"):
            return (self._last_ws.runs() if self._last_ws is not None else self.table).clone()

    def lifecycle(self):
        """Python-side ownership state; queries nothing on the device."""
        return self._own.state()

    def close(self):
        """Wait for the construction stream to drain, then refuse further calls. If the drain
        fails, the runner is poisoned and keeps the tensors of a failed call alive."""
        self._own.close()


class CoopRunner512(CoopRunnerCapacity):
    """runtime/ds41/moe_coop512.py:170 (default capacity 64 rows). ``run`` returns the runner's
    own output rows, overwritten by the next call (moe_coop512.py:248)."""
    DEFAULT_MAX_ROWS = 64
    OWNED_OUTPUT = False


class CoopRunner2048(CoopRunnerCapacity):
    """runtime/ds41/moe_coop2048.py:220 (default capacity 256 rows)."""
    DEFAULT_MAX_ROWS = 256


class CoopRunner3072(CoopRunnerCapacity):
    """runtime/ds41/moe_coop3072.py:261 (default capacity 512 rows)."""
    DEFAULT_MAX_ROWS = 512


@dataclasses.dataclass(frozen=True)
class WorkspaceLayout:
    """Device memory a capacity runner owns (moe_coop3072.py:120-152, read by its production owner
    as ``WorkspaceLayout().scratch_bytes``, native3072_runtime.py:134,146): the libevamx MoE
    workspace (``evamx_moe_workspace_bytes``) plus the runner's own output rows, fp16 routing
    weights, run table and prepare_routes workspace. Defaults are the reference's checkpoint
    shape (512 rows, H5120, I2304, top-6, up to 384 local experts); every field is a parameter
    here, and ``strict_rows`` None follows DS41_STRICT_BATCH / DS41_VERIFY_MAX_ROWS as the
    runners do."""

    max_rows: int = 512
    hidden: int = 5120
    inter: int = 2304
    topk: int = 6
    n_local: int = 384
    has_shared: bool = False
    strict_rows: int | None = None

    def __post_init__(self):
        for name in ("max_rows", "hidden", "inter", "topk", "n_local"):
            if type(getattr(self, name)) is not int or getattr(self, name) < 1:
                raise ValueError(f"{name} must be a positive integer")
        if self.hidden % 128 or self.inter % 128:
            raise ValueError("hidden and inter must be multiples of 128")

    @property
    def slots(self) -> int:
        return self.max_rows * self.topk

    @property
    def run_table_ints(self) -> int:
        """Length of the run table (moe_coop3072.py:97-106): 2 + 2 * slots + 1."""
        return 2 + 2 * self.slots + 1

    @property
    def moe_workspace_bytes(self) -> int:
        strict = (verification.moe_strict_rows(self.max_rows, self.topk) if self.strict_rows is None
                  else self.strict_rows)
        shape = ops.MoeShape(self.max_rows, self.hidden, self.inter, self.topk, self.n_local, int(self.has_shared),
                             0, 0, strict)
        n = ops.lib().evamx_moe_workspace_bytes(ctypes.byref(shape))
        if n == 0:
            raise ValueError("invalid MoE shape: " + ops.lib().evamx_last_error().decode())
        return n

    @property
    def scratch_bytes(self) -> int:
        return (self.moe_workspace_bytes + self.max_rows * self.hidden * 4 + self.slots * 2
                + self.run_table_ints * 4 + ops.prepare_routes_workspace_bytes(self.max_rows, self.topk))


def source_metadata() -> dict:
    """Build identity of the library behind these runners (moe_coop3072.py's source_metadata
    reports the reference extension's): hashes of the HIP sources and the C header (sorted by
    relative POSIX path), of the compile recipe and of the built library, the ABI version, and
    the arithmetic geometry a caller pins a target to."""
    from . import _lib, build
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    files = sorted([os.path.join(build.CSRC, f) for f in os.listdir(build.CSRC)
                    if f.endswith((".hip", ".hpp"))] + [os.path.join(root, "include", "evamx.h")],
                   key=lambda f: os.path.relpath(f, root).replace(os.sep, "/"))
    h = hashlib.sha256()
    for f in files:
        h.update(os.path.relpath(f, root).replace(os.sep, "/").encode())
        with open(f, "rb") as fh:
            h.update(fh.read())
    recipe = {"source_sha256": h.hexdigest(), "hipcc_flags": list(build.FLAGS), "arch": build.ARCH}
    build_sha = hashlib.sha256(json.dumps(recipe, sort_keys=True, separators=(",", ":")).encode()).hexdigest()
    lib_sha = None
    if os.path.exists(_lib.LIB_PATH):
        with open(_lib.LIB_PATH, "rb") as fh:
            lib_sha = hashlib.sha256(fh.read()).hexdigest()
    return {"source_sha256": recipe["source_sha256"], "build_sha256": build_sha, "library_sha256": lib_sha,
            "source_files": len(files), "hipcc_flags": list(build.FLAGS), "arch": build.ARCH,
            "abi_version": _lib.ABI_VERSION, "codebook": "MUL1", "K": list(RATES),
            "strict_batch": verification.strict_batch(), "verification_max_rows": verification.verification_max_rows(),
            "strict_max_rows": verification.STRICT_MOE_MAX_ROWS, "strict_max_slots": verification.STRICT_MOE_MAX_SLOTS,
            "max_topk": 32, "max_local_experts": 512, "graph_capture_supported": True,
            "output_ownership": "owned clone (CoopRunner2048/3072), borrowed rows (CoopRunner, CoopRunner512)"}
