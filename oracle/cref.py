"""ctypes front-end of the C oracle (oracle/msda_ref.c) — TEST INFRASTRUCTURE ONLY.

Used by tests/ (full-size second oracle) and by bench.py's CPU-baseline leg. The library is built
by ``make -C oracle`` (``__graft_entry__.build()`` runs it) into ``oracle/_build/``.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libmsda_oracle.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"C oracle not built: {LIB_PATH} (run `make -C oracle`)")
        lib = ctypes.CDLL(LIB_PATH)
        i32p = ctypes.POINTER(ctypes.c_int32)
        fp = ctypes.c_void_p
        lib.msda_oracle_fwd.argtypes = [fp, fp, fp, fp] + [ctypes.c_int] * 6 + [i32p, ctypes.c_int64, ctypes.c_int]
        lib.msda_oracle_fwd.restype = ctypes.c_int
        lib.msda_oracle_bwd.argtypes = [fp] * 7 + [ctypes.c_int] * 6 + [i32p, ctypes.c_int64, ctypes.c_int]
        lib.msda_oracle_bwd.restype = ctypes.c_int
        lib.msda_oracle_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _shapes(spatial_shapes):
    arr = np.ascontiguousarray(np.asarray(spatial_shapes, dtype=np.int32).reshape(-1))
    return arr, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def forward(value, spatial_shapes, loc, attn, threads=0):
    """f32 forward; value [B*H,S,D], loc [B,Q,H,L,P,2], attn [B,Q,H,L*P] -> [B,Q,H*D] f32."""
    lib = load()
    value = np.ascontiguousarray(value, np.float32)
    loc = np.ascontiguousarray(loc, np.float32)
    attn = np.ascontiguousarray(attn, np.float32)
    b, q, h, l, p, _ = loc.shape
    d = value.shape[-1]
    out = np.empty((b, q, h * d), np.float32)
    arr, sp = _shapes(spatial_shapes)
    rc = lib.msda_oracle_fwd(_ptr(value), _ptr(loc), _ptr(attn), _ptr(out), b, h, d, q, l, p, sp, value.shape[1], threads)
    if rc != 0:
        raise ValueError("msda_oracle_fwd rejected its arguments")
    return out


def backward(value, spatial_shapes, loc, attn, grad, threads=0):
    """f32 gradients (dvalue, dloc, dattn)."""
    lib = load()
    value = np.ascontiguousarray(value, np.float32)
    loc = np.ascontiguousarray(loc, np.float32)
    attn = np.ascontiguousarray(attn, np.float32)
    grad = np.ascontiguousarray(grad, np.float32)
    b, q, h, l, p, _ = loc.shape
    d = value.shape[-1]
    dv = np.empty_like(value)
    dl = np.empty_like(loc)
    da = np.empty_like(attn)
    arr, sp = _shapes(spatial_shapes)
    rc = lib.msda_oracle_bwd(_ptr(value), _ptr(loc), _ptr(attn), _ptr(grad), _ptr(dv), _ptr(dl), _ptr(da),
                             b, h, d, q, l, p, sp, value.shape[1], threads)
    if rc != 0:
        raise ValueError("msda_oracle_bwd rejected its arguments")
    return dv, dl, da


def max_threads():
    return load().msda_oracle_threads()
