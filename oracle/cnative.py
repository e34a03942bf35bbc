"""ctypes loader for the scalar C restatement ``oracle/exl3_oracle.c`` (test infrastructure).

Built by ``oracle/Makefile`` into ``oracle/_build/libexl3oracle.so`` (``__graft_entry__.build``
runs it). Used only by tests to cross-check ``oracle.exl3``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libexl3oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.evo_mul1_decode.restype = ctypes.c_uint16
        _lib.evo_mul1_decode.argtypes = [ctypes.c_uint32]
        _lib.evo_codebook.argtypes = [ctypes.c_void_p]
        _lib.evo_state_scalar.restype = ctypes.c_uint16
        _lib.evo_state_scalar.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        _lib.evo_states_group8.restype = ctypes.c_int
        _lib.evo_states_group8.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        _lib.evo_dequant.restype = ctypes.c_int
        _lib.evo_dequant.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        _lib.evo_had128.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def codebook() -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().evo_codebook(_ptr(out))
    return out.view(np.float16)


def states_scalar(words: np.ndarray, K: float) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.uint32)
    k2 = int(round(2 * K))
    return np.array([lib().evo_state_scalar(_ptr(w), k2, p) for p in range(256)], dtype=np.uint16)


def states_group8(words: np.ndarray, K: float) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.uint32)
    k2 = int(round(2 * K))
    out = np.empty(256, dtype=np.uint16)
    buf = np.empty(8, dtype=np.uint16)
    for t in range(0, 256, 8):
        if lib().evo_states_group8(_ptr(w), k2, t, _ptr(buf)):
            raise ValueError("group-of-8 form covers K <= 5 and half rates")
        out[t:t + 8] = buf
    return out


def dequant(trellis: np.ndarray, K: float) -> np.ndarray:
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    kt, nt, _ = t.shape
    out = np.empty((kt * 16, nt * 16), dtype=np.uint16)
    rc = lib().evo_dequant(_ptr(t), kt * 16, nt * 16, int(round(2 * K)), _ptr(out))
    if rc:
        raise ValueError("evo_dequant rejected the shape")
    return out.view(np.float16)


def had128(v: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty_like(x)
    lib().evo_had128(_ptr(x), _ptr(out), x.size // 128)
    return out
