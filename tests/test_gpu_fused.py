"""Parity of the fused-prologue op (msda_fused_fwd / msda_fused_bwd through the C ABI) on an MI355X.

The expected values are the prologue oracle (oracle/prologue_ref.py: locations and softmax weights
in f32 as ops.py:388-404 forms them, and the VJP in float64) composed with the core oracles: the
float64 NumPy one at reduced sizes, the f32 C one at the benchmark's full size. Tolerances are the
core's (``max|got - want| <= tol * max(1, max|want|)``): f32 forward 1e-5, gradients 1e-4; bf16
value 2e-2.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import msda_ref as R
from oracle import prologue_ref as PR
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import make_fused_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(_dev())


def _run_fused(value, shapes, ref, off, logits, grad, bf16=False, needs=(True, True, True, True)):
    v = _t(value)
    if bf16:
        v = v.to(torch.bfloat16)
    r, o, lg = _t(ref), _t(off), _t(logits)
    out = hip.ms_deform_attn_fused_forward(v, shapes, r, o, lg)
    grads = hip.ms_deform_attn_fused_backward(v, shapes, r, o, lg, _t(grad), needs=needs) if grad is not None else None
    torch.cuda.synchronize()
    return _np(out), None if grads is None else [_np(g) for g in grads]


def _oracle64(value, shapes, ref, off, logits, grad, p):
    loc, attn = PR.prologue(ref, off, logits, shapes, p)
    out = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    goff, glog, gref = PR.prologue_vjp(ref, off, logits, shapes, p, gl, ga)
    return out, (gv, gref, goff, glog)


def _check(got_out, got_grads, want_out, want_grads, bf16):
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(got_out, want_out, tf, "out")
    for name, g, w in zip(("grad_value", "grad_reference_points", "grad_sampling_offsets", "grad_attention_logits"),
                          got_grads, want_grads):
        assert_close(g, w, tg, name)


CASES = {
    # one 24x24 level, 2 points: the grouped forward with paired lanes (the Nano decoder's shape)
    "nano": dict(shapes=((24, 24),), heads=16, dim=16, points=2, queries=300),
    # two levels x 2 points: four samples per (query, head), the NS = 4 grouped forward
    "two_levels_p2": dict(shapes=((20, 30), (10, 15)), heads=8, dim=32, points=2, queries=200),
    # two levels x 4 points with a level too large for LDS: the per-query forward, L2 gathers
    "two_levels_p4": dict(shapes=((80, 80), (20, 20)), heads=16, dim=16, points=4, queries=150),
    # four levels x 4 points, 8 heads x 32 (the larger variants' decoder)
    "four_levels": dict(shapes=((40, 40), (20, 20), (10, 10), (5, 5)), heads=8, dim=32, points=4, queries=120),
    # the forward's staged head group fills the LDS (bf16: 4 heads x 32 x 40 x 16 x 2 B = 160 KB;
    # four heads per workgroup from 1024 queries)
    "lds_full": dict(shapes=((32, 40),), heads=16, dim=16, points=2, queries=1024),
}


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("ref_dim", [2, 4])
@pytest.mark.parametrize("case", sorted(CASES))
def test_fused_against_float64_oracle(case, ref_dim, bf16):
    c = CASES[case]
    _note(f"fused {case} ref_dim={ref_dim} bf16={bf16}")
    value, ref, off, logits, grad = make_fused_inputs(7, 2, c["heads"], c["dim"], c["queries"], c["shapes"], c["points"],
                                                      ref_dim, "bf16" if bf16 else "f32")
    out, grads = _run_fused(value, c["shapes"], ref, off, logits, grad, bf16)
    want_out, want_grads = _oracle64(value, c["shapes"], ref, off, logits, grad, c["points"])
    _check(out, grads, want_out, want_grads, bf16)


@pytest.mark.parametrize("ref_dim", [2, 4])
def test_fused_full_size_against_c_oracle(ref_dim):
    """The benchmark's config-2 shape (B=8, Q=3900, one 24x24 level, 16 heads x 16, 2 points) with
    the prologue fused, against the f32 C oracle, plus <G, out> = <dV, V>."""
    shapes = ((24, 24),)
    _note(f"fused full size ref_dim={ref_dim}")
    value, ref, off, logits, grad = make_fused_inputs(2, 8, 16, 16, 3900, shapes, 2, ref_dim)
    out, (gv, gref, goff, glog) = _run_fused(value, shapes, ref, off, logits, grad)
    loc, attn = PR.prologue(ref, off, logits, shapes, 2)
    assert_close(out, cref.forward(value, shapes, loc, attn), 1e-5, "out")
    cv, cl, ca = cref.backward(value, shapes, loc, attn, grad)
    w_off, w_log, w_ref = PR.prologue_vjp(ref, off, logits, shapes, 2, cl, ca)
    assert_close(gv, cv, 1e-4, "grad_value")
    assert_close(goff, w_off, 1e-4, "grad_sampling_offsets")
    assert_close(glog, w_log, 1e-4, "grad_attention_logits")
    assert_close(gref, w_ref, 1e-4, "grad_reference_points")
    inner = float(np.sum(out.astype(np.float64) * grad))
    assert math.isclose(float(np.sum(gv.astype(np.float64) * value)), inner, rel_tol=1e-4)


@pytest.mark.parametrize("bf16", [True, False], ids=["bf16", "f32"])
@pytest.mark.parametrize("ref_dim", [2, 4])
def test_fused_config3_size_against_c_oracle(ref_dim, bf16):
    """The benchmark's config-3 shape (B=8, Q=300, 80x80 + 20x20 levels, 16 heads x 16, 4 points;
    bf16 value as the workload has it, and f32) with the prologue fused: several levels, so the
    prologue and epilogue kernels run around the banded backward. Against the f32 C oracle on the
    same (bf16-rounded) values, plus <G, out> = <dV, V>."""
    shapes = ((80, 80), (20, 20))
    _note(f"fused config-3 size ref_dim={ref_dim} bf16={bf16}")
    value, ref, off, logits, grad = make_fused_inputs(3, 8, 16, 16, 300, shapes, 4, ref_dim, "bf16" if bf16 else "f32")
    out, (gv, gref, goff, glog) = _run_fused(value, shapes, ref, off, logits, grad, bf16)
    loc, attn = PR.prologue(ref, off, logits, shapes, 4)
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out, cref.forward(value, shapes, loc, attn), tf, "out")
    cv, cl, ca = cref.backward(value, shapes, loc, attn, grad)
    w_off, w_log, w_ref = PR.prologue_vjp(ref, off, logits, shapes, 4, cl, ca)
    assert_close(gv, cv, tg, "grad_value")
    assert_close(goff, w_off, tg, "grad_sampling_offsets")
    assert_close(glog, w_log, tg, "grad_attention_logits")
    assert_close(gref, w_ref, tg, "grad_reference_points")
    inner = float(np.sum(out.astype(np.float64) * grad))
    assert math.isclose(float(np.sum(gv.astype(np.float64) * value)), inner, rel_tol=1e-2 if bf16 else 1e-4)


@pytest.mark.parametrize("variant", [
    {"MSDA_FWD_GROUPED": "0"},          # per-query forward loop
    {"MSDA_FWD_PAIR": "0"},             # grouped forward without paired lanes
    {"MSDA_BWD_MAX_VEC": "16"},         # backward band kernel: one lane per (query, head)
    {"MSDA_BWD_MAX_VEC": "4"},          # four lanes per (query, head)
    {"MSDA_BWD_FORCE_BANDS": "1", "MSDA_BWD_BANDS": "5"},  # row bands: points straddle bands
], ids=lambda v: ",".join(f"{k}={x}" for k, x in v.items()))
def test_fused_kernel_variants(tune, variant):
    for k, x in variant.items():
        tune({k: x})
    shapes = ((24, 24), (12, 12))
    _note(f"fused variant {variant}")
    value, ref, off, logits, grad = make_fused_inputs(11, 2, 16, 16, 250, shapes, 2, 4)
    out, grads = _run_fused(value, shapes, ref, off, logits, grad)
    want_out, want_grads = _oracle64(value, shapes, ref, off, logits, grad, 2)
    _check(out, grads, want_out, want_grads, False)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("points,ref_dim", [(2, 4), (2, 2), (4, 4)])
def test_fused_in_kernel_and_row_paths_agree(tune, points, ref_dim, bf16):
    """One whole level: the band kernel forms locations and weights itself and writes the offset,
    logit and reference-point gradients (the in-kernel path); MSDA_FUSED_IN_KERNEL=0 forces the
    prologue and epilogue row kernels around the plain band kernel. Both agree with the float64
    oracle, and with each other to f32 rounding."""
    shapes = ((24, 24),)
    _note(f"fused in-kernel vs rows P={points} ref_dim={ref_dim} bf16={bf16}")
    value, ref, off, logits, grad = make_fused_inputs(17, 3, 16, 16, 333, shapes, points, ref_dim,
                                                      "bf16" if bf16 else "f32")
    want_out, want_grads = _oracle64(value, shapes, ref, off, logits, grad, points)
    runs = []
    for flag in (1, 0):
        tune({"MSDA_FUSED_IN_KERNEL": flag})
        runs.append(_run_fused(value, shapes, ref, off, logits, grad, bf16))
        _check(*runs[-1], want_out, want_grads, bf16)
    (out1, g1), (out0, g0) = runs
    assert np.array_equal(out1, out0), "the flag changes only the backward"
    for name, a, b in zip(("grad_value", "grad_reference_points", "grad_sampling_offsets", "grad_attention_logits"),
                          g1, g0):
        assert_close(a, b, 1e-5, name)


ROW_CASES = {
    # 9 samples per row (3 levels x 3 points): the 16-sample kernels; 6 heads: four (b, q) groups of
    # 54 threads per workgroup, and 8 lanes in the head tree with two of them zero
    "l3_p3_h6": dict(shapes=((12, 12), (6, 6), (3, 3)), heads=6, dim=16, points=3, queries=70),
    # 32 samples per row (4 levels x 8 points), two (b, q) groups per workgroup
    "l4_p8": dict(shapes=((16, 16), (8, 8), (4, 4), (2, 2)), heads=4, dim=16, points=8, queries=50),
    # 16 heads x 16 samples: one (b, q) group fills the workgroup
    "l4_p4_h16": dict(shapes=((16, 16), (8, 8), (4, 4), (2, 2)), heads=16, dim=16, points=4, queries=40),
    # 16 heads x 32 samples (512 threads per group) and 5 levels: past the per-sample kernels'
    # bounds, so the per-row kernels run either way
    "l4_p8_h16": dict(shapes=((16, 16), (8, 8), (4, 4), (2, 2)), heads=16, dim=16, points=8, queries=30),
    "l5_p2": dict(shapes=((16, 16), (8, 8), (4, 4), (2, 2), (1, 1)), heads=4, dim=16, points=2, queries=50),
    # power-of-two rows, whose softmax the per-sample kernels take across the row's lanes: 8 samples
    # (the config-3 shape's 2 levels x 4 points) and 2 samples (2 levels x 1 point)
    "l2_p4": dict(shapes=((20, 20), (10, 10)), heads=8, dim=16, points=4, queries=90),
    "l2_p1": dict(shapes=((20, 20), (10, 10)), heads=8, dim=16, points=1, queries=90),
}


@pytest.mark.parametrize("ref_dim", [2, 4])
@pytest.mark.parametrize("case", sorted(ROW_CASES))
def test_fused_row_kernels(tune, case, ref_dim):
    """Several levels: the prologue and epilogue run as kernels of their own around the band
    kernel. The kernels with one thread per sample (rows of at most 32 samples over at most 4
    levels) and those with one thread per row (MSDA_FUSED_PER_SAMPLE=0) give bit-identical
    reference-point, offset and logit gradients (grad_value within its run-to-run bound), matching
    the float64 oracle; some logits are masked (-inf)."""
    c = ROW_CASES[case]
    _note(f"fused row kernels {case} ref_dim={ref_dim}")
    value, ref, off, logits, grad = make_fused_inputs(15, 2, c["heads"], c["dim"], c["queries"], c["shapes"], c["points"],
                                                      ref_dim)
    logits[:, ::4, :, 1] = -np.inf
    out, grads = _run_fused(value, c["shapes"], ref, off, logits, grad)
    tune({"MSDA_FUSED_PER_SAMPLE": "0"})
    out0, grads0 = _run_fused(value, c["shapes"], ref, off, logits, grad)
    assert np.array_equal(out, out0)
    assert_close(grads[0], grads0[0], 1e-5, "grad_value")
    for name, g, g0 in zip(("grad_reference_points", "grad_sampling_offsets", "grad_attention_logits"), grads[1:], grads0[1:]):
        assert np.array_equal(g, g0), name
    want_out, want_grads = _oracle64(value, c["shapes"], ref, off, logits, grad, c["points"])
    _check(out, grads, want_out, want_grads, False)


def test_fused_three_points_four_heads():
    """Four heads, three points (n_points not a power of two: the box form divides), one small
    level; the epilogue sums grad_reference_points over four head lanes."""
    shapes = ((16, 16),)
    value, ref, off, logits, grad = make_fused_inputs(12, 3, 4, 16, 97, shapes, 3, 2)
    out, grads = _run_fused(value, shapes, ref, off, logits, grad)
    want_out, want_grads = _oracle64(value, shapes, ref, off, logits, grad, 3)
    _check(out, grads, want_out, want_grads, False)


@pytest.mark.parametrize("which", range(4))
def test_fused_single_gradient_requests(which):
    shapes = ((24, 24),)
    value, ref, off, logits, grad = make_fused_inputs(13, 2, 16, 16, 120, shapes, 2, 4)
    needs = tuple(i == which for i in range(4))
    _, grads = _run_fused(value, shapes, ref, off, logits, grad, needs=needs)
    _, want = _oracle64(value, shapes, ref, off, logits, grad, 2)
    for i, (g, w) in enumerate(zip(grads, want)):
        if i == which:
            assert_close(g, w, 1e-4, f"gradient {i}")
        else:
            assert g is None


def test_fused_masked_logits():
    """Logits of -inf (masked samples) get weight 0 and gradient 0, as jax.nn.softmax gives."""
    shapes = ((24, 24),)
    value, ref, off, logits, grad = make_fused_inputs(14, 1, 16, 16, 64, shapes, 4, 2)
    logits[:, ::3, :, 1] = -np.inf
    logits[:, 1::5, 2, :3] = -np.inf
    out, grads = _run_fused(value, shapes, ref, off, logits, grad)
    want_out, want_grads = _oracle64(value, shapes, ref, off, logits, grad, 4)
    assert np.isfinite(out).all()
    _check(out, grads, want_out, want_grads, False)
    assert (grads[3][:, ::3, :, 1] == 0).all()


def test_fused_matches_composed_torch_prologue():
    """Autograd through the fused op equals autograd through the prologue written in torch (f32,
    on the GPU) followed by the core op."""
    shapes = ((24, 24), (12, 12))
    value, ref, off, logits, grad = make_fused_inputs(15, 2, 16, 16, 200, shapes, 2, 4)
    leaves = [_t(x).requires_grad_(True) for x in (value, ref, off, logits)]
    out = hip.ms_deform_attn_fused(leaves[0], shapes, *leaves[1:])
    out.backward(_t(grad))
    fused = [_np(out)] + [_np(x.grad) for x in leaves]

    leaves2 = [_t(x).requires_grad_(True) for x in (value, ref, off, logits)]
    v, r, o, lg = leaves2
    loc = r[:, :, None, :, None, :2] + o / 2 * r[:, :, None, :, None, 2:] * 0.5
    attn = torch.softmax(lg, dim=-1)
    out2 = hip.ms_deform_attn_core_rows(v, shapes, loc, attn)
    out2.backward(_t(grad))
    composed = [_np(out2)] + [_np(x.grad) for x in leaves2]
    assert_close(fused[0], composed[0], 1e-5, "out")
    for name, a, b in zip(("value", "ref", "offsets", "logits"), fused[1:], composed[1:]):
        assert_close(a, b, 1e-4, f"grad {name}")


def test_fused_empty_queries():
    shapes = ((8, 8),)
    value, ref, off, logits, grad = make_fused_inputs(16, 2, 4, 8, 0, shapes, 2, 4)
    out, (gv, gref, goff, glog) = _run_fused(value, shapes, ref, off, logits, grad)
    assert out.shape == (2, 0, 32) and gref.shape == (2, 0, 1, 4) and goff.shape == (2, 0, 4, 1, 2, 2)
    assert (gv == 0).all()
