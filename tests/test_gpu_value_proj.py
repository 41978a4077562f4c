"""Parity of the value projection (msda_value_proj_fwd / _bwd through the C ABI) and of the
``MSDeformAttn`` module built on the fused kernels, on an MI355X.

Expected values: oracle/value_proj_ref.py (float64) for the projection; for the module, the same
module written with torch ops only (``F.linear``, ``masked_fill``, the prologue, ``F.grid_sample``
and the weighted sum) in float64 on the CPU. Tolerances: f32 forward 1e-5, gradients 1e-4 (the
projection sums 256-term f32 products, within that bound); bf16 2e-2.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import value_proj_ref as VP
from oracle.msda_ref import bf16_round
from rfdetr_jax_amd import MSDeformAttn
from rfdetr_jax_amd.value_proj import value_proj_backward, value_proj_forward
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(_dev())
    return t if dtype is None else t.to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy()


SHAPES = {
    "nano_memory": dict(b=2, s=576, k=256, h=16, d=16),   # 24x24 encoder memory, d_model 256
    "odd": dict(b=3, s=37, k=48, h=3, d=20),              # edge tiles in every dimension
    "base": dict(b=1, s=1700, k=256, h=8, d=32),          # 8 heads x 32 (larger variants)
    "odd_steps": dict(b=1, s=130, k=160, h=4, d=12),      # odd reduction step counts; 64 % D != 0
    "elementwise": dict(b=2, s=45, k=30, h=2, d=5),       # K, D not multiples of 4: element-wise kernels
    # divisors of 1 in the epilogue's (head, d) and (batch, position) splits, whose multiply-high
    # magic 2^32 has no 32-bit form
    "head_dim_1": dict(b=2, s=333, k=64, h=8, d=1),
    "len_in_1": dict(b=5, s=1, k=32, h=4, d=8),
}


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_value_proj_against_oracle(shape, masked, bf16):
    c = SHAPES[shape]
    _note(f"value_proj {shape} masked={masked} bf16={bf16}")
    rng = np.random.default_rng(31)
    x = rng.standard_normal((c["b"], c["s"], c["k"])).astype(np.float32)
    w = (rng.standard_normal((c["h"] * c["d"], c["k"])) / np.sqrt(c["k"])).astype(np.float32)
    bias = rng.standard_normal(c["h"] * c["d"]).astype(np.float32)
    mask = (rng.uniform(0, 1, (c["b"], c["s"])) < 0.2) if masked else None
    g = rng.standard_normal((c["b"] * c["h"], c["s"], c["d"])).astype(np.float32)
    if bf16:
        x, g = bf16_round(x), bf16_round(g)
    dt = torch.bfloat16 if bf16 else None
    tm = None if mask is None else _t(mask)
    out = value_proj_forward(_t(x, dt), _t(w), _t(bias), c["h"], tm)
    gx, gw, gb = value_proj_backward(_t(x, dt), _t(w), c["h"], _t(g, dt), tm)
    torch.cuda.synchronize()
    wq = bf16_round(w) if bf16 else w  # the product sees weight.astype(x.dtype)
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), VP.value_proj_rows(x, wq, bias, c["h"], mask), tf, "value")
    rx, rw, rb = VP.value_proj_rows_vjp(x, wq, c["h"], g, mask)
    assert_close(_np(gx), rx, tg, "grad_input")
    assert_close(_np(gw), rw, tg, "grad_weight")
    assert_close(_np(gb), rb, tg, "grad_bias")


def test_value_proj_no_bias_and_partial_requests():
    rng = np.random.default_rng(32)
    x = rng.standard_normal((2, 50, 64)).astype(np.float32)
    w = rng.standard_normal((64, 64)).astype(np.float32) / 8
    g = rng.standard_normal((16, 50, 8)).astype(np.float32)
    out = value_proj_forward(_t(x), _t(w), None, 8)
    assert_close(_np(out), VP.value_proj_rows(x, w, None, 8), 1e-5, "value")
    for needs in ((True, False, False), (False, True, False), (False, False, True)):
        got = value_proj_backward(_t(x), _t(w), 8, _t(g), None, needs)
        want = VP.value_proj_rows_vjp(x, w, 8, g)
        for i, (a, b) in enumerate(zip(got, want)):
            if needs[i]:
                assert_close(_np(a), b, 1e-4, f"gradient {i}")
            else:
                assert a is None


def _torch_module_reference(params, query, ref, inp, shapes, mask, n_heads, n_levels, n_points, grad):
    """MSDeformAttn (ops.py:338-411) written with torch ops only, float64 on the CPU."""
    import torch.nn.functional as F

    from oracle.msda_ref import level_offsets

    p = {k: torch.tensor(v.astype(np.float64), requires_grad=True) for k, v in params.items()}
    q = torch.tensor(query.astype(np.float64))
    r = torch.tensor(ref.astype(np.float64))
    x = torch.tensor(inp.astype(np.float64))
    b, lq, c = q.shape
    s = x.shape[1]
    value = F.linear(x, p["value_proj.weight"], p["value_proj.bias"])
    if mask is not None:
        value = value.masked_fill(torch.tensor(mask)[..., None], 0.0)
    logits = F.linear(q, p["attention_weights.weight"], p["attention_weights.bias"]).view(b, lq, n_heads, n_levels * n_points)
    off = F.linear(q, p["sampling_offsets.weight"], p["sampling_offsets.bias"]).view(b, lq, n_heads, n_levels, n_points, 2)
    if r.shape[-1] == 2:
        norm = torch.tensor([[w_, h_] for h_, w_ in shapes], dtype=torch.float64)
        loc = r[:, :, None, :, None, :] + off / norm[None, None, None, :, None, :]
    else:
        loc = r[:, :, None, :, None, :2] + off / n_points * r[:, :, None, :, None, 2:] * 0.5
    attn = torch.softmax(logits, -1)
    d = c // n_heads
    v = value.view(b, s, n_heads, d).permute(0, 2, 1, 3).reshape(b * n_heads, s, d)
    starts = level_offsets(shapes)
    out = torch.zeros(b * n_heads, d, lq, dtype=torch.float64)
    a_nl = attn.view(b, lq, n_heads, n_levels, n_points).permute(0, 2, 1, 3, 4).reshape(b * n_heads, lq, n_levels, n_points)
    for lvl, (hl, wl) in enumerate(shapes):
        v_l = v[:, starts[lvl]:starts[lvl + 1], :].transpose(1, 2).reshape(b * n_heads, d, hl, wl)
        grid = (2 * loc[:, :, :, lvl] - 1).permute(0, 2, 1, 3, 4).reshape(b * n_heads, lq, n_points, 2)
        sampled = F.grid_sample(v_l, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
        out = out + (sampled * a_nl[:, None, :, lvl, :]).sum(-1)
    out = out.view(b, n_heads, d, lq).permute(0, 3, 1, 2).reshape(b, lq, c)
    y = F.linear(out, p["output_proj.weight"], p["output_proj.bias"])
    y.backward(torch.tensor(grad.astype(np.float64)))
    return y.detach().numpy(), {k: t.grad.numpy() for k, t in p.items()}


@pytest.mark.parametrize("ref_dim", [2, 4])
def test_msdeform_attn_module_against_torch_module(ref_dim):
    """The whole module: value projection + mask + head split, prologue, sampling, output projection,
    forward and every parameter gradient, against the module written in torch ops."""
    torch.manual_seed(0)
    shapes = ((24, 24), (12, 12))
    n_heads, n_levels, n_points, d_model = 8, 2, 2, 64
    m = MSDeformAttn(d_model, n_levels, n_heads, n_points).to(_dev())
    rng = np.random.default_rng(33)
    with torch.no_grad():  # non-trivial offsets and attention projections (the upstream init zeroes them)
        m.sampling_offsets.weight.copy_(_t((rng.standard_normal(m.sampling_offsets.weight.shape) * 0.05).astype(np.float32)))
        m.attention_weights.weight.copy_(_t((rng.standard_normal(m.attention_weights.weight.shape) * 0.1).astype(np.float32)))
        m.value_proj.bias.copy_(_t((rng.standard_normal(d_model) * 0.1).astype(np.float32)))
    b, lq = 2, 50
    s = sum(h * w for h, w in shapes)
    query = rng.standard_normal((b, lq, d_model)).astype(np.float32)
    ref = rng.uniform(0.1, 0.9, (b, lq, 1, 2)).astype(np.float32)
    if ref_dim == 4:
        ref = np.concatenate([ref, rng.uniform(0.05, 0.4, (b, lq, 1, 2)).astype(np.float32)], -1)
    ref = np.ascontiguousarray(np.broadcast_to(ref, (b, lq, n_levels, ref_dim)))
    inp = rng.standard_normal((b, s, d_model)).astype(np.float32)
    mask = rng.uniform(0, 1, (b, s)) < 0.1
    grad = rng.standard_normal((b, lq, d_model)).astype(np.float32)
    out = m(_t(query), _t(ref), _t(inp), shapes, _t(mask))
    out.backward(_t(grad))
    params = {k: _np(v) for k, v in m.named_parameters()}
    want, want_grads = _torch_module_reference(params, query, ref, inp, shapes, mask, n_heads, n_levels, n_points, grad)
    assert_close(_np(out), want, 1e-5, "module output")
    for k, v in m.named_parameters():
        assert_close(_np(v.grad), want_grads[k], 1e-4, f"grad {k}")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_vector_and_elementwise_kernels_agree(tune, bf16):
    """The 16-byte operand kernels with 32- and 64-row tiles (MSDA_VP_BM) and the element-wise ones
    (MSDA_VP_SCALAR) on the same inputs, all against the oracle: they differ in tiling, staging and
    in how the bias gradient is formed."""
    rng = np.random.default_rng(34)
    b, s, k, h, d = 2, 300, 128, 8, 16
    x = rng.standard_normal((b, s, k)).astype(np.float32)
    w = (rng.standard_normal((h * d, k)) / np.sqrt(k)).astype(np.float32)
    bias = rng.standard_normal(h * d).astype(np.float32)
    mask = rng.uniform(0, 1, (b, s)) < 0.3
    g = rng.standard_normal((b * h, s, d)).astype(np.float32)
    if bf16:
        x, g = bf16_round(x), bf16_round(g)
    dt = torch.bfloat16 if bf16 else None
    wq = bf16_round(w) if bf16 else w
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    want = [VP.value_proj_rows(x, wq, bias, h, mask), *VP.value_proj_rows_vjp(x, wq, h, g, mask)]
    for mode in ("bm32", "bm64", "scalar"):
        if mode == "scalar":
            tune({"MSDA_VP_SCALAR": "1"})
        else:
            tune({"MSDA_VP_BM": mode[2:]})
        out = value_proj_forward(_t(x, dt), _t(w), _t(bias), h, _t(mask))
        got = [out, *value_proj_backward(_t(x, dt), _t(w), h, _t(g, dt), _t(mask))]
        torch.cuda.synchronize()
        for name, a, ref, tol in zip(("value", "grad_input", "grad_weight", "grad_bias"), got, want, (tf, tg, tg, tg)):
            assert_close(_np(a), ref, tol, f"{name} {mode}")


@pytest.mark.parametrize("seed", range(8))
def test_msdeform_attn_module_random_shapes(seed):
    """The whole module on random draws: 1-4 levels of 1-30 rows and columns, 1-8 heads, head_dim
    4-32, 1-4 points, point or box reference points, a padding mask or none, against the module in
    torch ops (float64, CPU), output and every parameter gradient."""
    rng = np.random.default_rng(600 + seed)
    n_levels = int(rng.integers(1, 5))
    shapes = tuple((int(rng.integers(1, 31)), int(rng.integers(1, 31))) for _ in range(n_levels))
    n_heads, n_points = int(rng.choice([1, 2, 4, 8])), int(rng.integers(1, 5))
    d_model = n_heads * int(rng.choice([4, 8, 12, 16, 32]))
    ref_dim, masked = (2, 4)[int(rng.integers(0, 2))], bool(rng.integers(0, 2))
    b, lq = int(rng.integers(1, 3)), int(rng.integers(1, 80))
    _note(f"module random seed={seed} shapes={shapes} heads={n_heads} points={n_points} d_model={d_model} ref_dim={ref_dim} "
          f"masked={masked} b={b} lq={lq}")
    torch.manual_seed(seed)
    m = MSDeformAttn(d_model, n_levels, n_heads, n_points).to(_dev())
    with torch.no_grad():
        m.sampling_offsets.weight.copy_(_t((rng.standard_normal(m.sampling_offsets.weight.shape) * 0.05).astype(np.float32)))
        m.attention_weights.weight.copy_(_t((rng.standard_normal(m.attention_weights.weight.shape) * 0.1).astype(np.float32)))
        m.value_proj.bias.copy_(_t((rng.standard_normal(d_model) * 0.1).astype(np.float32)))
    s = sum(h * w for h, w in shapes)
    query = rng.standard_normal((b, lq, d_model)).astype(np.float32)
    ref = rng.uniform(0.1, 0.9, (b, lq, 1, 2)).astype(np.float32)
    if ref_dim == 4:
        ref = np.concatenate([ref, rng.uniform(0.05, 0.4, (b, lq, 1, 2)).astype(np.float32)], -1)
    ref = np.array(np.broadcast_to(ref, (b, lq, n_levels, ref_dim)))  # a writable copy
    inp = rng.standard_normal((b, s, d_model)).astype(np.float32)
    mask = (rng.uniform(0, 1, (b, s)) < 0.1) if masked else None
    grad = rng.standard_normal((b, lq, d_model)).astype(np.float32)
    out = m(_t(query), _t(ref), _t(inp), shapes, None if mask is None else _t(mask))
    out.backward(_t(grad))
    params = {k: _np(v) for k, v in m.named_parameters()}
    want, want_grads = _torch_module_reference(params, query, ref, inp, shapes, mask, n_heads, n_levels, n_points, grad)
    assert_close(_np(out), want, 1e-5, "module output")
    for k, v in m.named_parameters():
        assert_close(_np(v.grad), want_grads[k], 1e-4, f"grad {k}")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_value_proj_misaligned_tensors(bf16):
    """Input and grad_value views one element into their buffers (K and D multiples of 4, so only
    the alignment keeps them off the 16-byte tile kernels): the element-wise kernels, against the
    oracle."""
    rng = np.random.default_rng(35)
    b, s, k, h, d = 2, 70, 64, 4, 16
    x = rng.standard_normal((b, s, k)).astype(np.float32)
    w = (rng.standard_normal((h * d, k)) / 8).astype(np.float32)
    bias = rng.standard_normal(h * d).astype(np.float32)
    g = rng.standard_normal((b * h, s, d)).astype(np.float32)
    if bf16:
        x, g = bf16_round(x), bf16_round(g)
    dt = torch.bfloat16 if bf16 else torch.float32
    xb = torch.zeros(x.size + 1, dtype=dt, device=_dev())
    xb[1:] = _t(x.ravel(), dt)
    gb_ = torch.zeros(g.size + 1, dtype=dt, device=_dev())
    gb_[1:] = _t(g.ravel(), dt)
    xv, gvv = xb[1:].view(b, s, k), gb_[1:].view(b * h, s, d)
    assert xv.data_ptr() % 16 != 0 and gvv.data_ptr() % 16 != 0
    out = value_proj_forward(xv, _t(w), _t(bias), h)
    gx, gw, gb = value_proj_backward(xv, _t(w), h, gvv)
    torch.cuda.synchronize()
    wq = bf16_round(w) if bf16 else w
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), VP.value_proj_rows(x, wq, bias, h), tf, "value")
    rx, rw, rb = VP.value_proj_rows_vjp(x, wq, h, g)
    assert_close(_np(gx), rx, tg, "grad_input")
    assert_close(_np(gw), rw, tg, "grad_weight")
    assert_close(_np(gb), rb, tg, "grad_bias")
