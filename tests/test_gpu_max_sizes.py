"""The core op at the size limits msda.h states, on an MI355X, through size-independent checks.

The float64 oracle cannot run at these sizes, so the checks are what the mathematics fixes whatever
the size:
* forward at 2^30 value elements per slice (a 16384 x 1024 level at head_dim 64, 4 GiB in f32, the
  most that index arithmetic inside a slice allows): bilinear interpolation reproduces a function
  that is linear in the pixel coordinates exactly, so with value[y, x, c] = a_c x + b_c y + c_c
  and weights that sum to one, every output channel is sum_p A_p (a_c ix_p + b_c iy_p) + c_c for
  samples whose four corners lie inside the level; the samples sit near the far corner of the
  level, where the element offsets are largest;
* forward and backward at the tallest level (32000 rows, the largest the C ABI accepts) by 128
  columns at head_dim 64 (262 M elements per slice; one image row of the backward's f64
  accumulator and its staged value rows fill most of the LDS): the output is linear in the value
  and in the weights, so <G, out> = <dV, V> = <dA, A> (sums in float64 on the GPU);
* a level too wide for one image row of the backward's f64 accumulator to fit in LDS is refused
  with MSDA_ERR_UNSUPPORTED, its forward still runs;
* a level whose image row fits only beside a shorter point list (more scan passes per band)
  against the float64 oracle;
* the self-attention at 2048 and 4096 rows against the float64 oracle.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from rfdetr_jax_amd import _native
from rfdetr_jax_amd import ops as hip

pytestmark = pytest.mark.gpu


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _gen(seed):
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    return gen


def test_largest_slice_forward_reproduces_a_linear_map():
    h, w, d = 16384, 1024, 64
    assert h * w * d == 1 << 30
    _note(f"max size forward {h}x{w} head_dim {d}")
    dev = torch.device("cuda:0")
    gen = _gen(21)
    a, b, c = (torch.randn(d, device=dev, generator=gen) * s for s in (1e-3, 1e-4, 1.0))
    value = (a * torch.arange(w, device=dev, dtype=torch.float32)[None, :, None]
             + b * torch.arange(h, device=dev, dtype=torch.float32)[:, None, None] + c).reshape(1, h * w, d)
    q, p = 512, 2
    # locations in the last 64 rows and columns, at least one pixel from the border
    loc = torch.empty(1, q, 1, 1, p, 2, device=dev)
    loc[..., 0] = (w - 64 + torch.rand(1, q, 1, 1, p, device=dev, generator=gen) * 62 + 0.5) / w
    loc[..., 1] = (h - 64 + torch.rand(1, q, 1, 1, p, device=dev, generator=gen) * 62 + 0.5) / h
    attn = torch.softmax(torch.randn(1, q, 1, p, device=dev, generator=gen), -1)
    out = hip.ms_deform_attn_forward(value, ((h, w),), loc, attn)
    torch.cuda.synchronize()
    ix = loc[..., 0].double().reshape(q, p) * w - 0.5  # pixel coordinates, ops.py:83-84
    iy = loc[..., 1].double().reshape(q, p) * h - 0.5
    A = attn.double().reshape(q, p)
    want = ((A * ix).sum(-1)[:, None] * a.double() + (A * iy).sum(-1)[:, None] * b.double()
            + A.sum(-1)[:, None] * c.double())
    err = float((out.double().reshape(q, d) - want).abs().max())
    scale = max(1.0, float(want.abs().max()))
    _note(f"max size forward: max|err| {err:.3e} scale {scale:.3e}")
    assert err <= 1e-5 * scale
    del value


def test_tallest_level_identities():
    shapes = ((32000, 128),)
    _note(f"max size fwd+bwd {shapes} head_dim 64")
    dev = torch.device("cuda:0")
    gen = _gen(11)
    value = torch.randn(1, 32000 * 128, 64, device=dev, generator=gen)
    q, p = 4000, 4
    loc = torch.rand(1, q, 1, 1, p, 2, device=dev, generator=gen) * 1.2 - 0.1
    attn = torch.softmax(torch.randn(1, q, 1, p, device=dev, generator=gen), -1)
    grad = torch.randn(1, q, 64, device=dev, generator=gen)
    out = hip.ms_deform_attn_forward(value, shapes, loc, attn)
    gv, gl, ga = hip.ms_deform_attn_backward(value, shapes, loc, attn, grad)
    torch.cuda.synchronize()
    inner = float((out.double() * grad.double()).sum())
    dv_v = float((gv.double() * value.double()).sum())
    da_a = float((ga.double() * attn.double()).sum())
    _note(f"<G,out> {inner:.9e} <dV,V> {dv_v:.9e} <dA,A> {da_a:.9e}")
    assert math.isfinite(inner) and abs(inner) > 0
    assert math.isclose(dv_v, inner, rel_tol=1e-5)
    assert math.isclose(da_a, inner, rel_tol=1e-5)
    assert bool(torch.isfinite(gl).all())
    del value, gv


def test_level_too_wide_for_the_backward_is_refused():
    """One image row of 4096 cells x 64 channels needs 2 MiB of f64 accumulator: the forward runs
    (L2 gathers), the backward raises with the library's message."""
    shapes = ((8, 4096),)
    dev = torch.device("cuda:0")
    gen = _gen(12)
    value = torch.randn(1, 8 * 4096, 64, device=dev, generator=gen)
    loc = torch.rand(1, 100, 1, 1, 2, 2, device=dev, generator=gen)
    attn = torch.softmax(torch.randn(1, 100, 1, 2, device=dev, generator=gen), -1)
    grad = torch.randn(1, 100, 64, device=dev, generator=gen)
    out = hip.ms_deform_attn_forward(value, shapes, loc, attn)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    with pytest.raises(_native.MsdaError) as err:
        hip.ms_deform_attn_backward(value, shapes, loc, attn, grad)
    assert err.value.code == _native.ERR_UNSUPPORTED
    _note(f"refused: {err.value}")


def test_wide_level_with_a_shorter_point_list_against_oracle():
    """A 150-column level at head_dim 64 (f32): one image row of the band (its f64 accumulator and two
    staged value rows) leaves room for a list of 256 queries' points, not the usual 2048, so the band
    scans the 3000 queries in 12 passes. Against the float64 oracle."""
    from oracle import msda_ref as R
    from rfdetr_jax_amd.workloads import make_inputs
    from tests._util import assert_close

    shapes = ((6, 150),)
    value, loc, attn, grad = make_inputs(31, 1, 2, 64, 3000, shapes, 4, uniform_locations=True)
    dev = torch.device("cuda:0")
    v, lc, a, g = (torch.from_numpy(x).to(dev) for x in (value, loc, attn, grad))
    out = hip.ms_deform_attn_forward(v, shapes, lc, a)
    gv, gl, ga = hip.ms_deform_attn_backward(v, shapes, lc, a, g)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv.cpu().numpy(), rv, 1e-4, "grad_value")
    assert_close(gl.cpu().numpy(), rl, 1e-4, "grad_loc")
    assert_close(ga.cpu().numpy(), ra, 1e-4, "grad_attn")


@pytest.mark.parametrize("length,head_dim,bf16,masked", [(2048, 64, False, True), (4096, 32, True, False), (4096, 64, False, False)])
def test_long_attention_against_oracle(length, head_dim, bf16, masked):
    """The chunked self-attention kernels far past the decoder's 300 rows (32 to 64 key chunks per
    query block, the forward's reference score moving many times) against the float64 oracle."""
    import numpy as np

    from oracle import attention_ref as AT
    from oracle.msda_ref import bf16_round
    from rfdetr_jax_amd.attention import scaled_dot_product_attention
    from tests._util import assert_close

    _note(f"long attention L={length} D={head_dim} bf16={bf16} masked={masked}")
    rng = np.random.default_rng(length + head_dim)
    q, k, v, g = (rng.standard_normal((1, 2, length, head_dim)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    mask = None
    if masked:
        mask = rng.uniform(0, 1, (length, length)) < 0.3
        mask[7] = True
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (torch.from_numpy(x).to(dev).to(dt).requires_grad_(True) for x in (q, k, v))
    out = scaled_dot_product_attention(tq, tk, tv, None if mask is None else torch.from_numpy(mask).to(dev))
    out.backward(torch.from_numpy(g).to(dev).to(dt))
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out.float().detach().cpu().numpy(), AT.sdpa(q, k, v, mask), tf, "out")
    for name, t, want in zip("qkv", (tq, tk, tv), AT.sdpa_vjp(q, k, v, g, mask)):
        assert_close(t.grad.float().cpu().numpy(), want, tg, f"grad_{name}")
