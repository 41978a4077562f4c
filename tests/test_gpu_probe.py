"""The device probes behind the benchmark's LDS rooflines (include/msda_probe.h) on an MI355X:
their outputs are the closed forms their documentation states."""

from __future__ import annotations

import ctypes

import pytest
import torch

from rfdetr_jax_amd import _native

pytestmark = pytest.mark.gpu


def test_lds_atomic_probe_sums():
    """Every LDS accumulator receives one 1.0 per repetition from one lane, so each thread's sum of
    16 of them is 16 * reps, and the total is msda_probe_lds_atomic_ops."""
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    lib = _native.lib()
    blocks, reps = 7, 5
    out = torch.full((blocks * 256,), -1.0, dtype=torch.float64, device="cuda:0")
    assert lib.msda_probe_lds_atomic(ctypes.c_void_p(out.data_ptr()), blocks, reps, None) == 0
    torch.cuda.synchronize()
    assert torch.all(out == 16.0 * reps)
    assert lib.msda_probe_lds_atomic_ops(blocks, reps) == blocks * 256 * 16 * reps
    assert lib.msda_probe_lds_atomic(None, blocks, reps, None) == -1


def test_lds_atomic_f32_probe_sums():
    """The f32 probe's accumulators: one 1.0f per repetition each, so 16 * reps per thread (exact)."""
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    lib = _native.lib()
    blocks, reps = 5, 3
    out = torch.full((blocks * 256,), -1.0, dtype=torch.float32, device="cuda:0")
    assert lib.msda_probe_lds_atomic_f32(ctypes.c_void_p(out.data_ptr()), blocks, reps, None) == 0
    torch.cuda.synchronize()
    assert torch.all(out == 16.0 * reps)
    assert lib.msda_probe_lds_atomic_f32(None, blocks, reps, None) == -1


def test_lds_read_probe_runs():
    """The read probe fills its output (one word per thread) and reports 8 KB per thread-repetition
    group as documented."""
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    lib = _native.lib()
    blocks, reps = 3, 4
    out = torch.zeros(blocks * 256, dtype=torch.int32, device="cuda:0")
    assert lib.msda_probe_lds_read(ctypes.c_void_p(out.data_ptr()), blocks, reps, None) == 0
    torch.cuda.synchronize()
    assert lib.msda_probe_lds_read_bytes(blocks, reps) == blocks * 256 * reps * 8 * 16
    assert lib.msda_probe_lds_read(None, blocks, reps, None) == -1
