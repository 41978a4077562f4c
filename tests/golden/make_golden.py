"""Generate the golden fixtures under tests/golden/ (``python tests/golden/make_golden.py``).

The reference (RF-DETR-JAX) is pure JAX and JAX is not installed here, so the fixtures come from
this repository's float64 NumPy oracle (oracle/msda_ref.py). Before a fixture is written, its
forward is checked against torch ``F.grid_sample`` (bilinear, zeros, align_corners=False) and its
gradients against torch autograd through grid_sample, both in float64, so a fixture never records
an oracle mistake. Inputs are stored with the expected outputs; GPU tests read them as data.

Each ``.npz`` holds: value (f32; bf16-representable for bf16 cases), loc, attn, grad (f32),
shapes (int32 [L,2]), out, grad_value, grad_loc, grad_attn (float64 oracle results stored as
float32, far inside every tolerance), and ``meta`` (a JSON
string: name, seed, value dtype, how the inputs were drawn).
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import msda_ref as R  # noqa: E402

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "rf-detr-jax_amd"))
from rfdetr_jax_amd.workloads import make_inputs  # noqa: E402


def torch_reference(value, shapes, loc, attn, grad):
    """Forward and VJP via torch grid_sample + autograd in float64 (independent of the oracle)."""
    import torch
    import torch.nn.functional as F

    b, q, h, l, p, _ = loc.shape
    d = value.shape[-1]
    v = torch.tensor(np.asarray(value, np.float64), requires_grad=True)
    lc = torch.tensor(np.asarray(loc, np.float64), requires_grad=True)
    a = torch.tensor(np.asarray(attn, np.float64), requires_grad=True)
    offsets = R.level_offsets(shapes)
    out = torch.zeros(b * h, d, q, dtype=torch.float64)
    a_nl = a.reshape(b, q, h, l, p).permute(0, 2, 1, 3, 4).reshape(b * h, q, l, p)
    for lvl, (hl, wl) in enumerate(shapes):
        v_l = v[:, offsets[lvl] : offsets[lvl + 1], :].transpose(1, 2).reshape(b * h, d, hl, wl)
        grid = 2 * lc[:, :, :, lvl] - 1  # [B,Q,H,P,2]
        grid = grid.permute(0, 2, 1, 3, 4).reshape(b * h, q, p, 2)
        sampled = F.grid_sample(v_l, grid, mode="bilinear", padding_mode="zeros", align_corners=False)  # [N,D,Q,P]
        out = out + (sampled * a_nl[:, None, :, lvl, :]).sum(-1)
    out = out.reshape(b, h, d, q).permute(0, 3, 1, 2).reshape(b, q, h * d)
    out.backward(torch.tensor(np.asarray(grad, np.float64)))
    return out.detach().numpy(), v.grad.numpy(), lc.grad.numpy(), a.grad.numpy()


def _case(name, value, shapes, loc, attn, grad, meta, check_torch=True):
    out = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    if check_torch:
        t_out, t_gv, t_gl, t_ga = torch_reference(value, shapes, loc, attn, grad)
        scale = max(1.0, float(np.abs(t_out).max()))
        assert np.abs(out - t_out).max() <= 1e-5 * scale, name
        for mine, theirs in ((gv, t_gv), (gl, t_gl), (ga, t_ga)):
            assert np.abs(mine - theirs).max() <= 1e-4 * max(1.0, float(np.abs(theirs).max())), name
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        value=np.asarray(value, np.float32), loc=np.asarray(loc, np.float32), attn=np.asarray(attn, np.float32),
        grad=np.asarray(grad, np.float32), shapes=np.asarray(shapes, np.int32).reshape(-1, 2),
        out=out.astype(np.float32), grad_value=gv.astype(np.float32), grad_loc=gl.astype(np.float32),
        grad_attn=ga.astype(np.float32), meta=json.dumps(meta),
    )
    print(f"wrote {name}.npz")


def main():
    # Known answers of the reference's tests (tests/test_ops.py:22-54), in the rows layout.
    # 1) pixel centres of a 2x2 map [[1,2],[3,4]]: grid (-0.5,-0.5) -> 1, (0.5,0.5) -> 4.
    value = np.array([1, 2, 3, 4], np.float32).reshape(1, 4, 1)
    loc = np.array([[0.25, 0.25], [0.75, 0.75]], np.float32).reshape(1, 2, 1, 1, 1, 2)
    _case("kat_pixel_centres", value, ((2, 2),), loc, np.ones((1, 2, 1, 1), np.float32),
          np.ones((1, 2, 1), np.float32), {"source": "tests/test_ops.py:22-29", "expect": [1.0, 4.0]})
    # 2) out of bounds: grid (5,5) on ones -> 0.
    _case("kat_zero_pad", np.ones((1, 4, 1), np.float32), ((2, 2),), np.full((1, 1, 1, 1, 1, 2), 3.0, np.float32),
          np.ones((1, 1, 1, 1), np.float32), np.ones((1, 1, 1), np.float32),
          {"source": "tests/test_ops.py:32-36", "expect": [0.0]})
    # 3) midpoint of [[0, 4]] (H=1, W=2) at grid (0,0) -> 2.
    _case("kat_midpoint", np.array([0, 4], np.float32).reshape(1, 2, 1), ((1, 2),),
          np.full((1, 1, 1, 1, 1, 2), 0.5, np.float32), np.ones((1, 1, 1, 1), np.float32),
          np.ones((1, 1, 1), np.float32), {"source": "tests/test_ops.py:39-43", "expect": [2.0]})
    # 4) uniform weights over two points of arange(4) 2x2 -> 1.5.
    _case("kat_mean_of_points", np.arange(4, dtype=np.float32).reshape(1, 4, 1), ((2, 2),),
          np.array([[0.25, 0.25], [0.75, 0.75]], np.float32).reshape(1, 1, 1, 1, 2, 2),
          np.full((1, 1, 1, 2), 0.5, np.float32), np.ones((1, 1, 1), np.float32),
          {"source": "tests/test_ops.py:46-54", "expect": [1.5]})

    # The reference's fused-sampler parity shape (tests/test_ops.py:225-248), f32 and bf16 value.
    for dtype in ("f32", "bf16"):
        rng = np.random.default_rng(3)
        shapes = ((8, 16), (4, 8))
        b, q, h, l, p, d = 2, 70, 2, 2, 3, 8
        s = sum(hh * ww for hh, ww in shapes)
        value = rng.standard_normal((b * h, s, d)).astype(np.float32)
        if dtype == "bf16":
            value = R.bf16_round(value)
        loc = rng.uniform(-0.1, 1.1, (b, q, h, l, p, 2)).astype(np.float32)
        attn = rng.uniform(0, 1, (b, q, h, l * p)).astype(np.float32)
        grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
        _case(f"two_level_{dtype}", value, shapes, loc, attn, grad,
              {"source": "tests/test_ops.py:225-248 shape", "seed": 3, "value_dtype": dtype})

    # The reference's matmul-vs-gather shape with locations in U[-0.2, 1.2] (tests/test_ops.py:112-124).
    rng = np.random.default_rng(0)
    b, h, d, hh, ww, q, p = 2, 4, 8, 7, 5, 11, 3
    value = rng.standard_normal((b * h, hh * ww, d)).astype(np.float32)
    loc = (rng.uniform(0, 1, (b, q, h, 1, p, 2)) * 1.4 - 0.2).astype(np.float32)
    attn = rng.uniform(0, 1, (b, q, h, p)).astype(np.float32)
    grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
    _case("odd_map_7x5", value, ((hh, ww),), loc, attn, grad, {"source": "tests/test_ops.py:112-124 shape", "seed": 0})

    # Exact pixel centres and exact cell corners (floor at integers), plus far / huge positions.
    rng = np.random.default_rng(11)
    shapes = ((8, 8),)
    b, q, h, p, d = 1, 48, 2, 4, 4
    value = rng.standard_normal((b * h, 64, d)).astype(np.float32)
    grid_pts = (np.arange(-2, 11) / 8.0).astype(np.float32)  # pixel edges: loc = k/8 -> ix = k - 0.5
    centres = ((np.arange(-1, 10) + 0.5) / 8.0).astype(np.float32)  # pixel centres -> integer ix
    pool = np.concatenate([grid_pts, centres, np.array([-3.0, 4.0, 1e6, -1e6, 0.0, 1.0], np.float32)])
    loc = rng.choice(pool, size=(b, q, h, 1, p, 2)).astype(np.float32)
    attn = rng.uniform(0, 1, (b, q, h, p)).astype(np.float32)
    grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
    # torch's float64 grid differs from the f32 grid only by rounding; at exact integers the
    # one-sided derivatives of the two can differ, so only the forward is cross-checked here.
    out = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    t_out = torch_reference(value, shapes, loc, attn, grad)[0]
    assert np.abs(out - t_out).max() <= 1e-6
    _case("integer_and_far_positions", value, shapes, loc, attn, grad,
          {"seed": 11, "note": "locations on pixel edges/centres, far outside, and +-1e6"}, check_torch=False)

    # Head dims other than 16 and more levels/points.
    for d in (1, 3, 32):
        rng = np.random.default_rng(100 + d)
        shapes = ((6, 9), (3, 5))
        b, q, h, p = 2, 17, 3, 2
        s = sum(x * y for x, y in shapes)
        value = rng.standard_normal((b * h, s, d)).astype(np.float32)
        loc = rng.uniform(-0.2, 1.2, (b, q, h, 2, p, 2)).astype(np.float32)
        attn = rng.uniform(0, 1, (b, q, h, 2 * p)).astype(np.float32)
        grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
        _case(f"head_dim_{d}", value, shapes, loc, attn, grad, {"seed": 100 + d})

    rng = np.random.default_rng(7)
    shapes = ((16, 16), (8, 8), (4, 4), (2, 2))
    b, q, h, p, d = 1, 40, 4, 4, 16
    s = sum(x * y for x, y in shapes)
    value = rng.standard_normal((b * h, s, d)).astype(np.float32)
    ref = rng.uniform(0, 1, (b, q, 2))
    loc = (ref[:, :, None, None, None, :] + rng.normal(0, 0.1, (b, q, h, 4, p, 2))).astype(np.float32)
    logits = rng.standard_normal((b, q, h, 4 * p))
    attn = (np.exp(logits) / np.exp(logits).sum(-1, keepdims=True)).astype(np.float32)
    grad = rng.standard_normal((b, q, h * d)).astype(np.float32)
    _case("four_levels", value, shapes, loc, attn, grad, {"seed": 7, "note": "RF-DETR default n_levels=4, n_points=4"})

    # Small version of the Nano decoder shape (configs 0-2: 24x24, 16 heads x 16, 2 points).
    value, loc, attn, grad = make_inputs(0, 1, 4, 16, 40, ((24, 24),), 2)
    _case("nano_small", value, ((24, 24),), loc, attn, grad, {"seed": 0, "draw": "make_inputs(0, B=1, H=4, Q=40)"})


if __name__ == "__main__":
    main()
