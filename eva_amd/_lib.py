"""ctypes binding of libevamx.so (the C ABI declared in include/evamx.h).

torch is imported first so that its HIP runtime is the one the library binds to (both carry the
SONAME libamdhip64.so.7). There is no fallback: if the library is missing or a call fails, an
exception is raised.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library resolves against)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libevamx.so")
ABI_VERSION = 5

EVAMX_OK, EVAMX_EINVAL, EVAMX_ELAUNCH, EVAMX_ENOSPACE = 0, -1, -2, -3
DTYPE_F16, DTYPE_BF16 = 0, 1
SCORE_SIGMOID, SCORE_SQRT_SOFTPLUS = 0, 1
ERR_EXPERT_RANGE, ERR_RATE = 1, 2
STRICT_MAX_ROWS, STRICT_MAX_SLOTS = 64, 256      # EVAMX_STRICT_MAX_ROWS / EVAMX_STRICT_MAX_SLOTS

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class MoeShape(ctypes.Structure):
    _fields_ = [("rows_max", _i32), ("hidden", _i32), ("inter", _i32), ("topk", _i32),
                ("n_local", _i32), ("has_shared", _i32), ("ksplit_gu", _i32), ("ksplit_down", _i32),
                ("strict_rows", _i32)]                                              # ABI 5


class MoeArgs(ctypes.Structure):
    _fields_ = [("shape", MoeShape), ("rows", _i32), ("x", _vp), ("x_dtype", _i32), ("x_stride", _i32),
                ("logits", _vp), ("sel_bias", _vp), ("n_logits", _i32), ("score_fn", _i32),
                ("route_scale", _f32), ("sel", _vp), ("weights", _vp), ("rw_fp16", _vp),
                ("min_expert", _i32), ("max_expert", _i32), ("tables", _vp), ("k2_per_expert", _vp),
                ("bits", _f32), ("shared", _vp), ("shared_bits", _f32), ("limit", _f32),
                ("out", _vp), ("out_stride", _i32), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
                ("events", _vp), ("residual", _vp), ("residual_stride", _i32), ("gate_w", _vp),
                ("bits_down", _f32), ("k2_down_per_expert", _vp), ("shared_bits_down", _f32),
                ("shared_gate_w", _vp)]


class EvamxError(RuntimeError):
    pass


_lib = None

# name -> (restype, argtypes)
_SIGNATURES = {
    "evamx_last_error": (ctypes.c_char_p, []),
    "evamx_abi_version": (ctypes.c_int, []),
    "evamx_exl3_dequant": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _f32, _vp, _vp]),
    "evamx_exl3_linear_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "evamx_exl3_linear": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp, _f32,
                                         _vp, _vp, ctypes.c_size_t, _vp]),
    "evamx_router_logits": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int,
                                           ctypes.c_int, _vp, _vp]),
    "evamx_route_topk": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32,
                                        _vp, _vp, _vp, _vp]),
    "evamx_prepare_routes_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "evamx_prepare_routes": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            _vp, _vp, ctypes.c_size_t, _vp]),
    "evamx_prepare_routes_flags_ptr": (_vp, [_vp]),
    "evamx_moe_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(MoeShape)]),
    "evamx_moe_workspace_init": (ctypes.c_int, [ctypes.POINTER(MoeShape), _vp, _vp]),
    "evamx_moe_forward": (ctypes.c_int, [ctypes.POINTER(MoeArgs), _vp]),
    "evamx_moe_forward_static": (ctypes.c_int, [ctypes.POINTER(MoeArgs), _vp]),
    "evamx_moe_runs_ptr": (_vp, [ctypes.POINTER(MoeShape), _vp]),
    "evamx_moe_flags_ptr": (_vp, [ctypes.POINTER(MoeShape), _vp]),
    "evamx_moe_logits_ptr": (_vp, [ctypes.POINTER(MoeShape), _vp]),
    "evamx_moe_rotated_ptr": (_vp, [ctypes.POINTER(MoeShape), _vp]),
    "evamx_bench_decode": (ctypes.c_int, [_f32, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "evamx_bench_read": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]),
}

EXPORTS = tuple(_SIGNATURES)


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise EvamxError(f"{LIB_PATH} is missing: build it with `python -m eva_amd.build` "
                             "(or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.evamx_abi_version() != ABI_VERSION:
            raise EvamxError("libevamx ABI version mismatch; rebuild the library")
        _lib = handle
    return _lib


def check(rc: int, what: str):
    if rc != EVAMX_OK:
        msg = lib().evamx_last_error().decode(errors="replace")
        raise EvamxError(f"{what} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
