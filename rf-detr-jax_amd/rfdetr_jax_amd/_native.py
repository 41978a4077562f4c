"""ctypes binding of the HIP library's C ABI (include/msda.h).

There is no CPU fallback: if the library is missing, :func:`lib` raises, and every op that
needs it fails loudly.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

from .build import LIB_PATH

DTYPE_F32 = 0
DTYPE_BF16 = 1

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_LAUNCH = -3
ERR_DEVICE = -4

#: Every function include/msda.h declares, with its ctypes signature.
_I = ctypes.c_int
_P = ctypes.c_void_p
_I32P = ctypes.POINTER(ctypes.c_int32)
_I64 = ctypes.c_int64
_DIMS = [_I] * 6 + [_I32P, _I32P, _I64]  # batch .. n_points, spatial_shapes, level_start_index, len_value
SIGNATURES = {
    "msda_version": ([], ctypes.c_char_p),
    "msda_last_error": ([], ctypes.c_char_p),
    "msda_set_tuning": ([ctypes.c_char_p, ctypes.c_char_p], _I),
    "msda_fwd": ([_P, _I, _P, _P, _P, _I] + _DIMS + [_P], _I),
    "msda_fwd_sampler": ([_P, _I, _P, _P, _P, _I, _I] + _DIMS + [_P], _I),
    "msda_bwd_workspace_size": (list(_DIMS), _I64),
    "msda_bwd": ([_P, _I, _P, _P, _P, _I, _P, _P, _P] + _DIMS + [_P, _I64, _P], _I),
    "msda_bwd_sampler": ([_P, _I, _P, _P, _P, _I, _P, _P, _P, _I] + _DIMS + [_P, _I64, _P], _I),
    "msda_bwd_noalloc": ([_P, _I, _P, _P, _P, _I, _P, _P, _P] + _DIMS + [_P], _I),
    "msda_fused_fwd": ([_P, _I, _P, _I, _P, _P, _P, _I] + _DIMS + [_P], _I),
    "msda_fused_bwd_workspace_size": ([_I] * 7 + [_I32P, _I32P, _I64], _I64),
    "msda_fused_bwd": ([_P, _I, _P, _I, _P, _P, _P, _I, _P, _P, _P, _P] + _DIMS + [_P, _I64, _P], _I),
    "msda_grid_sample_fwd": ([_P, _I, _P, _I, _P] + [_I] * 7 + [_P], _I),
    "msda_grid_sample_bwd": ([_P, _I, _P, _I, _P, _P, _P] + [_I] * 7 + [_P], _I),
    "msda_value_proj_fwd": ([_P, _I, _P, _P, _P, _P] + [_I] * 5 + [_P], _I),
    "msda_value_proj_bwd_workspace_size": ([_I] * 5, _I64),
    "msda_value_proj_bwd": ([_P, _I, _P, _P, _P, _P, _P, _P] + [_I] * 5 + [_P, _I64, _P], _I),
    "msda_attention_fwd": ([_P, _P, _P, _I, _P, _P] + [_I] * 5 + [_P, _P, _P], _I),
    "msda_attention_bwd": ([_P, _P, _P, _P, _P, _P, _I, _P, _P, _P] + [_I] * 5 + [_P, _P, _P], _I),
    "msda_attention_fwd_dropout": ([_P, _P, _P, _I, _P, _P] + [_I] * 5 + [_P, _P, ctypes.c_float, ctypes.c_uint64, _P], _I),
    "msda_attention_bwd_dropout": ([_P, _P, _P, _P, _P, _P, _I, _P, _P, _P] + [_I] * 5
                                   + [_P, _P, ctypes.c_float, ctypes.c_uint64, _P], _I),
    "msda_attention_dropout_keep": ([_I] * 4 + [ctypes.c_float, ctypes.c_uint64, _P, _P], _I),
    # include/msda_probe.h
    "msda_probe_lds_read": ([_P, _I, _I, _P], _I),
    "msda_probe_lds_read_bytes": ([_I, _I], _I64),
    "msda_probe_lds_atomic": ([_P, _I, _I, _P], _I),
    "msda_probe_lds_atomic_f32": ([_P, _I, _I, _P], _I),
    "msda_probe_lds_atomic_ops": ([_I, _I], _I64),
}

GRID_COORDS = 0
GRID_UNIT_POINTS = 1
PADDING = {"zeros": 0, "border": 1}
SAMPLE_BILINEAR = 0
SAMPLE_NEAREST = 1

_lock = threading.Lock()
_lib = None


class MsdaError(RuntimeError):
    """A failed library call; ``code`` is the MSDA_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"msda error {code}: {message}")
        self.code = code


def lib(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = path or os.environ.get("MSDA_LIBRARY", LIB_PATH)
        if not os.path.exists(target):
            raise RuntimeError(
                f"HIP library not found at {target}; build it with __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). There is no CPU fallback."
            )
        handle = ctypes.CDLL(target)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if path is None:
            _lib = handle
        return handle


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().msda_last_error().decode("utf-8", "replace")
        raise MsdaError(rc, msg)


@contextlib.contextmanager
def tuning(knobs: dict):
    """Override launch-tuning knobs (``{"MSDA_BWD_BANDS": 7, ...}``) for the duration of a block;
    the library reads them from the environment only once, so this is how a process switches
    launch variants (benchmarks, tests)."""
    set_ = []
    try:
        for name, value in knobs.items():
            check(lib().msda_set_tuning(name.encode(), str(value).encode()))
            set_.append(name)
        yield
    finally:
        for name in set_:
            lib().msda_set_tuning(name.encode(), None)
