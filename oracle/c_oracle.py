"""ctypes wrapper of the C online-softmax restatement (``oracle/attn_online.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libattn_oracle.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        i64 = ctypes.c_int64
        lib.attn_online_fwd.argtypes = [dp, dp, dp, dp, dp, i64, i64, i64, ctypes.c_int, i64]
        lib.attn_online_fwd.restype = ctypes.c_int
        lib.attn_online_bwd.argtypes = [dp, dp, dp, dp, dp, dp, dp, dp, dp, i64, i64, i64, ctypes.c_int]
        lib.attn_online_bwd.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def fwd(q, k, v, causal=False, tile=32):
    """Online-softmax forward, fp64. Returns (O, LSE)."""
    lib = load()
    q, k, v = _f64(q), _f64(k), _f64(v)
    b, h, t, d = q.shape
    o = np.empty_like(q)
    lse = np.empty((b, h, t))
    rc = lib.attn_online_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), b * h, t, d, int(causal), tile)
    if rc:
        raise RuntimeError(f"attn_online_fwd failed ({rc})")
    return o, lse


def bwd(q, k, v, o, do, lse, causal=False):
    """Recompute backward, fp64. Returns (dQ, dK, dV)."""
    lib = load()
    q, k, v, o, do, lse = (_f64(a) for a in (q, k, v, o, do, lse))
    b, h, t, d = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    rc = lib.attn_online_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse),
                             _ptr(dq), _ptr(dk), _ptr(dv), b * h, t, d, int(causal))
    if rc:
        raise RuntimeError(f"attn_online_bwd failed ({rc})")
    return dq, dk, dv
