"""Every sampler name the reference's dispatcher accepts (src/rfdetr_jax/models/ops.py:235-238,
:277-280: "gather", "gather-f32", "matmul", "auto", "pallas", plus this library's "hip") runs the
HIP kernels end to end through autograd, in f32 and bf16, against the float64 oracle.

The reference computes one function with every sampler; its samplers differ only in bf16 rounding
points (the kernels keep f32 throughout, which is within the bf16 tolerance below). Tolerances as
in test_gpu_parity: f32 1e-5 (output) and 1e-4 (gradients); bf16 values compared against f32 math
on the bf16-rounded values with 2e-2 (tests/test_ops.py:238 of the reference).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import msda_ref as R
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu

SHAPES = ((24, 24), (12, 12))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("sampler", ["gather", "gather-f32", "matmul", "auto", "pallas", "hip"])
def test_sampler_names_run_the_hip_path_with_autograd(sampler, dtype):
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    sys.stderr.write(f"[gpu] sampler={sampler} dtype={dtype}\n")
    sys.stderr.flush()
    dev = torch.device("cuda:0")
    bf16 = dtype == "bf16"
    value, loc, attn, grad = make_inputs(7, 2, 4, 16, 333, SHAPES, 2)
    if bf16:
        value = R.bf16_round(value)
    v = torch.from_numpy(value).to(dev)
    if bf16:
        v = v.to(torch.bfloat16)
    v.requires_grad_(True)
    lc = torch.from_numpy(loc).to(dev).requires_grad_(True)
    a = torch.from_numpy(attn).to(dev).requires_grad_(True)
    g = torch.from_numpy(grad).to(dev)
    out = hip.ms_deform_attn_core_rows(v, SHAPES, lc, a, sampler)
    assert out.is_cuda and out.dtype == torch.float32 and tuple(out.shape) == (2, 333, 64)
    (out * g).sum().backward()
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out.detach().cpu().numpy(), R.ms_deform_attn_core_rows(value, SHAPES, loc, attn), tf, f"{sampler} out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, SHAPES, loc, attn, grad)
    assert v.grad.dtype == v.dtype  # grad_value in the value dtype (deform_pallas.py:175)
    assert_close(v.grad.float().cpu().numpy(), rv, tg, f"{sampler} grad_value")
    assert_close(lc.grad.cpu().numpy(), rl, tg, f"{sampler} grad_loc")
    assert_close(a.grad.cpu().numpy(), ra, tg, f"{sampler} grad_attn")


def test_unknown_sampler_name_is_rejected_like_the_reference():
    v = torch.zeros(2, 720, 16, device="cuda")
    with pytest.raises(ValueError, match="unknown sampler"):
        hip.ms_deform_attn_core_rows(v, SHAPES, torch.zeros(1, 3, 2, 2, 2, 2, device="cuda"),
                                     torch.zeros(1, 3, 2, 4, device="cuda"), "bilinear")
