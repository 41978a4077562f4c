"""Pin the MSDeformAttn prologue oracle (oracle/prologue_ref.py) before trusting it.

Checks, none of which retypes the oracle's formulas:
* torch float64 autograd through torch's own softmax and broadcast arithmetic (the VJP);
* the full chain prologue -> F.grid_sample -> weighted sum under torch autograd, against the
  prologue oracle composed with the core oracle (forward and every gradient);
* closed forms: zero offsets give the reference point exactly; offsets of whole level sizes move a
  2-dim point by exact steps along x and y; a box offset of 2*P*k moves by k box widths; equal
  logits give 1/(L*P); softmax is invariant to a shift of one (query, head)'s logits; its VJP sums
  to zero per (query, head); grad_reference_points of 2-dim points is the sum of grad_loc over heads
  and points.
Planted mistakes (normaliser stacked as (H, W), the 0.5 of the box form dropped, a softmax over the
head axis instead of the sample axis) are shown to fail the closed forms.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import msda_ref as R
from oracle import prologue_ref as PR
from tests._util import assert_close


def _case(seed, ref_dim, shapes=((6, 10), (3, 5)), b=2, q=7, h=4, p=3, d=4):
    rng = np.random.default_rng(seed)
    n_levels = len(shapes)
    s = sum(x * y for x, y in shapes)
    value = rng.standard_normal((b * h, s, d)).astype(np.float32)
    if ref_dim == 2:
        ref = rng.uniform(0.05, 0.95, (b, q, n_levels, 2)).astype(np.float32)
        off = rng.normal(0.0, 1.5, (b, q, h, n_levels, p, 2)).astype(np.float32)
    else:
        ref = np.concatenate([rng.uniform(0.1, 0.9, (b, q, n_levels, 2)), rng.uniform(0.05, 0.5, (b, q, n_levels, 2))],
                             axis=-1).astype(np.float32)
        off = rng.normal(0.0, 2.0, (b, q, h, n_levels, p, 2)).astype(np.float32)
    logits = rng.normal(0.0, 2.0, (b, q, h, n_levels * p)).astype(np.float32)
    grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
    return value, shapes, ref, off, logits, grad, p


def _torch_prologue(ref, off, logits, shapes, n_points):
    """The prologue written with torch ops (autograd derives the VJP)."""
    import torch

    ref_dim = ref.shape[-1]
    if ref_dim == 2:
        norm = torch.tensor([[w, h] for h, w in shapes], dtype=ref.dtype)
        loc = ref[:, :, None, :, None, :] + off / norm[None, None, None, :, None, :]
    else:
        loc = ref[:, :, None, :, None, :2] + off / n_points * ref[:, :, None, :, None, 2:] * 0.5
    return loc, torch.softmax(logits, dim=-1)


@pytest.mark.parametrize("ref_dim", [2, 4])
@pytest.mark.parametrize("seed", [0, 1])
def test_prologue_vjp_matches_torch_autograd(ref_dim, seed):
    import torch

    _, shapes, ref, off, logits, _, p = _case(seed, ref_dim)
    rng = np.random.default_rng(100 + seed)
    g_loc = rng.standard_normal(off.shape)
    g_attn = rng.standard_normal(logits.shape)
    tr = torch.tensor(ref.astype(np.float64), requires_grad=True)
    to = torch.tensor(off.astype(np.float64), requires_grad=True)
    tl = torch.tensor(logits.astype(np.float64), requires_grad=True)
    loc, attn = _torch_prologue(tr, to, tl, shapes, p)
    ((loc * torch.tensor(g_loc)).sum() + (attn * torch.tensor(g_attn)).sum()).backward()
    gofs, glog, gref = PR.prologue_vjp(ref, off, logits, shapes, p, g_loc, g_attn)
    assert_close(gofs, to.grad.numpy(), 1e-12, "grad_offsets")
    assert_close(glog, tl.grad.numpy(), 1e-6, "grad_logits")  # oracle weights are f32
    assert_close(gref, tr.grad.numpy(), 1e-12, "grad_reference_points")
    # forward: f32 oracle against the f64 torch formula
    loc32, attn32 = PR.prologue(ref, off, logits, shapes, p)
    assert_close(loc32, loc.detach().numpy(), 1e-6, "loc")
    assert_close(attn32, attn.detach().numpy(), 1e-6, "attn")


@pytest.mark.parametrize("ref_dim", [2, 4])
def test_full_chain_matches_torch_autograd(ref_dim):
    """prologue -> grid_sample -> weighted sum, all under torch float64 autograd."""
    import torch
    import torch.nn.functional as F

    value, shapes, ref, off, logits, grad, p = _case(5, ref_dim)
    b, q, h, n_levels, _, _ = off.shape
    d = value.shape[-1]
    tv = torch.tensor(value.astype(np.float64), requires_grad=True)
    tr = torch.tensor(ref.astype(np.float64), requires_grad=True)
    to = torch.tensor(off.astype(np.float64), requires_grad=True)
    tl = torch.tensor(logits.astype(np.float64), requires_grad=True)
    loc, attn = _torch_prologue(tr, to, tl, shapes, p)
    starts = R.level_offsets(shapes)
    out = torch.zeros(b * h, d, q, dtype=torch.float64)
    a_nl = attn.reshape(b, q, h, n_levels, p).permute(0, 2, 1, 3, 4).reshape(b * h, q, n_levels, p)
    for lvl, (hl, wl) in enumerate(shapes):
        v_l = tv[:, starts[lvl] : starts[lvl + 1], :].transpose(1, 2).reshape(b * h, d, hl, wl)
        grid = (2 * loc[:, :, :, lvl] - 1).permute(0, 2, 1, 3, 4).reshape(b * h, q, p, 2)
        sampled = F.grid_sample(v_l, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
        out = out + (sampled * a_nl[:, None, :, lvl, :]).sum(-1)
    out = out.reshape(b, h, d, q).permute(0, 3, 1, 2).reshape(b, q, h * d)
    out.backward(torch.tensor(grad.astype(np.float64)))

    loc32, attn32 = PR.prologue(ref, off, logits, shapes, p)
    want_out = R.ms_deform_attn_core_rows(value, shapes, loc32, attn32)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc32, attn32, grad)
    gofs, glog, gref = PR.prologue_vjp(ref, off, logits, shapes, p, gl, ga)
    assert_close(want_out, out.detach().numpy(), 1e-5, "out")
    assert_close(gv, tv.grad.numpy(), 1e-4, "grad_value")
    assert_close(gofs, to.grad.numpy(), 1e-4, "grad_offsets")
    assert_close(glog, tl.grad.numpy(), 1e-4, "grad_logits")
    assert_close(gref, tr.grad.numpy(), 1e-4, "grad_reference_points")


# --------------------------------------------------------------------------------------------
# closed forms, written as checks on any prologue implementation so planted mistakes can be run
# through them


def _check_zero_offsets(fn):
    _, shapes, ref, off, logits, _, p = _case(2, 2)
    loc, _ = fn(ref, np.zeros_like(off), logits, shapes, p)
    assert np.array_equal(loc, np.broadcast_to(ref[:, :, None, :, None, :], loc.shape))
    _, shapes, ref4, off4, logits4, _, p = _case(2, 4)
    loc4, _ = fn(ref4, np.zeros_like(off4), logits4, shapes, p)
    assert np.array_equal(loc4, np.broadcast_to(ref4[:, :, None, :, None, :2], loc4.shape))


def _check_whole_level_steps(fn):
    """Offsets of (k*W_l, m*H_l) move a 2-dim point by exactly (k, m) (levels are not square)."""
    shapes = ((6, 10), (3, 5))
    ref = np.full((1, 1, 2, 2), 0.25, np.float32)
    off = np.zeros((1, 1, 1, 2, 1, 2), np.float32)
    for lvl, (hl, wl) in enumerate(shapes):
        off[0, 0, 0, lvl, 0] = (2.0 * wl, -1.0 * hl)
    loc, _ = fn(ref, off, np.zeros((1, 1, 1, 2), np.float32), shapes, 1)
    assert np.array_equal(loc[0, 0, 0, :, 0], np.array([[2.25, -0.75], [2.25, -0.75]], np.float32))


def _check_box_steps(fn):
    """A box offset of 2*P*k moves the centre by k box widths / heights."""
    shapes = ((6, 10),)
    p = 4
    ref = np.array([0.5, 0.25, 0.25, 0.125], np.float32).reshape(1, 1, 1, 4)
    off = np.zeros((1, 1, 1, 1, p, 2), np.float32)
    off[..., 0] = 2 * p * 1.0
    off[..., 1] = 2 * p * -2.0
    loc, _ = fn(ref, off, np.zeros((1, 1, 1, p), np.float32), shapes, p)
    assert np.array_equal(loc[0, 0, 0, 0], np.tile(np.array([0.75, 0.0], np.float32), (p, 1)))


def _check_softmax_forms(fn):
    _, shapes, ref, off, logits, _, p = _case(3, 2)
    lp = logits.shape[-1]
    _, attn = fn(ref, off, np.full_like(logits, 0.7), shapes, p)
    assert np.allclose(attn, 1.0 / lp, rtol=1e-6, atol=0)
    _, a1 = fn(ref, off, logits, shapes, p)
    shift = np.arange(logits.shape[2], dtype=np.float32)[None, None, :, None] * 3.0
    _, a2 = fn(ref, off, logits + shift, shapes, p)
    assert np.allclose(a1, a2, rtol=1e-5, atol=1e-7)
    assert np.allclose(a1.sum(-1), 1.0, atol=1e-6)


CHECKS = [_check_zero_offsets, _check_whole_level_steps, _check_box_steps, _check_softmax_forms]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_closed_forms(check):
    check(PR.prologue)


def test_vjp_invariants():
    _, shapes, ref, off, logits, _, p = _case(4, 2)
    rng = np.random.default_rng(9)
    g_loc = rng.standard_normal(off.shape)
    g_attn = rng.standard_normal(logits.shape)
    gofs, glog, gref = PR.prologue_vjp(ref, off, logits, shapes, p, g_loc, g_attn)
    # zero up to the f32 rounding of the weights' sum (sum_j y_j = 1 within ~1e-7)
    assert np.abs(glog.sum(-1)).max() < 1e-6
    assert np.allclose(gref, g_loc.sum(axis=(2, 4)), rtol=0, atol=1e-12)
    # grad_offsets * (W, H) recovers grad_loc
    norm = np.array([[w, h] for h, w in shapes], np.float64)
    assert np.allclose(gofs * norm[None, None, None, :, None, :], g_loc, rtol=1e-14, atol=0)


def _swapped_normaliser(ref, off, logits, shapes, p):
    return PR.prologue(ref, off, logits, tuple((w, h) for h, w in shapes), p)


def _dropped_half(ref, off, logits, shapes, p):
    if ref.shape[-1] == 4:
        ref = ref.copy()
        ref[..., 2:] *= 2.0
    return PR.prologue(ref, off, logits, shapes, p)


def _softmax_over_heads(ref, off, logits, shapes, p):
    loc, _ = PR.prologue(ref, off, logits, shapes, p)
    x = logits.astype(np.float32)
    e = np.exp(x - x.max(axis=2, keepdims=True))
    return loc, (e / e.sum(axis=2, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("mistake", [_swapped_normaliser, _dropped_half, _softmax_over_heads], ids=lambda m: m.__name__)
def test_planted_mistakes_are_caught(mistake):
    failed = 0
    for check in CHECKS:
        try:
            check(mistake)
        except AssertionError:
            failed += 1
    assert failed > 0, f"{mistake.__name__} passed every closed-form check"
