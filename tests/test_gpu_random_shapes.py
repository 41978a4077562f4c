"""Seeded random shapes through msda_fwd / msda_bwd against the float64 oracle, on an MI355X.

Each seed draws 1-4 levels of 1-40 rows and columns, 1-16 heads, head_dim 1-64, 1-8 points,
1-400 queries, batch 1-3, f32 or bf16 values, and locations either clustered around reference
points or uniform over [-0.1, 1.1]^2 (many corners outside the map). Both sizes are small enough
for the float64 oracle (oracle/msda_ref.py) to finish in well under a second. The launch planner
picks whatever plan the shape gets: whole levels or bands, query blocks and partial sums, lanes
per query, head groups, staged or gathered levels. Tolerances are the contract's
(``max|got - want| <= tol * max(1, max|want|)``): f32 forward 1e-5 and gradients 1e-4, bf16 2e-2.
A second set of draws runs each of the reference's sampler names, whose forward on a bf16 map is
held to 2e-6 of the oracle's restatement of that sampler (as in test_gpu_samplers).
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


def _draw(seed):
    rng = np.random.default_rng(7000 + seed)
    levels = int(rng.integers(1, 5))
    shapes = tuple((int(rng.integers(1, 41)), int(rng.integers(1, 41))) for _ in range(levels))
    return dict(
        shapes=shapes,
        heads=int(rng.choice([1, 2, 3, 4, 5, 8, 16])),
        dim=int(rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 48, 64])),
        points=int(rng.integers(1, 9)),
        queries=int(rng.integers(1, 401)),
        batch=int(rng.integers(1, 4)),
        bf16=bool(rng.integers(0, 2)),
        uniform=bool(rng.integers(0, 2)),
    )


@pytest.mark.parametrize("seed", range(24))
def test_random_shape_against_oracle(seed):
    c = _draw(seed)
    sys.stderr.write(f"[gpu] random shape seed={seed} {c}\n")
    sys.stderr.flush()
    value, loc, attn, grad = make_inputs(seed, c["batch"], c["heads"], c["dim"], c["queries"], c["shapes"], c["points"],
                                         value_dtype="bf16" if c["bf16"] else "f32", uniform_locations=c["uniform"])
    dev = torch.device("cuda:0")
    v = torch.from_numpy(value).to(dev)
    if c["bf16"]:
        v = v.to(torch.bfloat16)
    lc, a, g = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (loc, attn, grad))
    out = hip.ms_deform_attn_forward(v, c["shapes"], lc, a)
    gv, gl, ga = hip.ms_deform_attn_backward(v, c["shapes"], lc, a, g)
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if c["bf16"] else (1e-5, 1e-4)
    assert_close(out.float().cpu().numpy(), R.ms_deform_attn_core_rows(value, c["shapes"], loc, attn), tf, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, c["shapes"], loc, attn, grad)
    assert_close(gv.float().cpu().numpy(), rv, tg, "grad_value")
    assert_close(gl.cpu().numpy(), rl, tg, "grad_loc")
    assert_close(ga.cpu().numpy(), ra, tg, "grad_attn")


@pytest.mark.parametrize("seed", range(12))
def test_random_shape_named_sampler(seed):
    """The same draws through each reference sampler name (autograd over ms_deform_attn_core_rows):
    the forward against the oracle's restatement of that sampler's rounding points and pixel
    coordinates, the gradients against the f32 VJP at its coordinates."""
    c = _draw(100 + seed)
    sampler = hip.SAMPLERS[seed % len(hip.SAMPLERS)]
    sys.stderr.write(f"[gpu] random shape sampler={sampler} seed={seed} {c}\n")
    sys.stderr.flush()
    value, loc, attn, grad = make_inputs(100 + seed, c["batch"], c["heads"], c["dim"], c["queries"], c["shapes"], c["points"],
                                         value_dtype="bf16" if c["bf16"] else "f32", uniform_locations=c["uniform"])
    dev = torch.device("cuda:0")
    v = torch.from_numpy(value).to(dev)
    if c["bf16"]:
        v = v.to(torch.bfloat16)
    v.requires_grad_(True)
    lc = torch.from_numpy(np.ascontiguousarray(loc)).to(dev).requires_grad_(True)
    a = torch.from_numpy(np.ascontiguousarray(attn)).to(dev).requires_grad_(True)
    g = torch.from_numpy(grad).to(dev)
    out = hip.ms_deform_attn_core_rows(v, c["shapes"], lc, a, sampler)
    (out * g).sum().backward()
    torch.cuda.synchronize()
    tf, tg = (2e-6, 2e-2) if c["bf16"] else (1e-5, 1e-4)
    want = R.ms_deform_attn_core_rows_sampler(value, c["shapes"], loc, attn, sampler, c["bf16"])
    assert_close(out.detach().cpu().numpy(), want, tf, f"{sampler} out")
    vjp = R.ms_deform_attn_core_rows_vjp_pallas if sampler == "pallas" else R.ms_deform_attn_core_rows_vjp
    rv, rl, ra = vjp(value, c["shapes"], loc, attn, grad)
    assert_close(v.grad.float().cpu().numpy(), rv, tg, f"{sampler} grad_value")
    assert_close(lc.grad.cpu().numpy(), rl, tg, f"{sampler} grad_loc")
    assert_close(a.grad.cpu().numpy(), ra, tg, f"{sampler} grad_attn")


@pytest.mark.parametrize("seed", range(16))
def test_random_shape_fused_prologue(seed):
    """The fused-prologue op (msda_fused_fwd / msda_fused_bwd) on random draws with point (2-dim) or
    box (4-dim) reference points, against the prologue oracle composed with the core's float64
    oracle: one level takes the band kernel's in-kernel prologue when it fits, several levels the
    prologue and epilogue kernels (per sample for rows of up to 32 samples over up to 4 levels,
    per row otherwise)."""
    from oracle import prologue_ref as PR
    from rfdetr_jax_amd.workloads import make_fused_inputs

    c = _draw(200 + seed)
    ref_dim = 2 if seed % 2 == 0 else 4
    sys.stderr.write(f"[gpu] random shape fused seed={seed} ref_dim={ref_dim} {c}\n")
    sys.stderr.flush()
    value, ref, off, logits, grad = make_fused_inputs(200 + seed, c["batch"], c["heads"], c["dim"], c["queries"], c["shapes"],
                                                      c["points"], ref_dim, "bf16" if c["bf16"] else "f32")
    dev = torch.device("cuda:0")
    v = torch.from_numpy(value).to(dev)
    if c["bf16"]:
        v = v.to(torch.bfloat16)
    r, o, lg, g = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (ref, off, logits, grad))
    out = hip.ms_deform_attn_fused_forward(v, c["shapes"], r, o, lg)
    gv, gref, goff, glog = hip.ms_deform_attn_fused_backward(v, c["shapes"], r, o, lg, g)
    torch.cuda.synchronize()
    loc, attn = PR.prologue(ref, off, logits, c["shapes"], c["points"])
    want = R.ms_deform_attn_core_rows(value, c["shapes"], loc, attn)
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, c["shapes"], loc, attn, grad)
    roff, rlog, rref = PR.prologue_vjp(ref, off, logits, c["shapes"], c["points"], rl, ra)
    tf, tg = (2e-2, 2e-2) if c["bf16"] else (1e-5, 1e-4)
    assert_close(out.float().cpu().numpy(), want, tf, "out")
    assert_close(gv.float().cpu().numpy(), rv, tg, "grad_value")
    assert_close(gref.cpu().numpy(), rref, tg, "grad_reference_points")
    assert_close(goff.cpu().numpy(), roff, tg, "grad_sampling_offsets")
    assert_close(glog.cpu().numpy(), rlog, tg, "grad_attention_logits")


@pytest.mark.parametrize("seed", range(12))
def test_random_shape_value_projection(seed):
    """The value projection (msda_value_proj_fwd / _bwd) on random [B, S, C] -> H x D shapes: C and
    D multiples of 4 or not (the 16-byte MFMA tile kernel or the element-wise one), a padding mask
    or none, f32 or bf16, against the float64 oracle (oracle/value_proj_ref.py)."""
    from oracle import value_proj_ref as VP
    from oracle.msda_ref import bf16_round
    from rfdetr_jax_amd.value_proj import value_proj_backward, value_proj_forward

    rng = np.random.default_rng(300 + seed)
    b, s = int(rng.integers(1, 4)), int(rng.integers(1, 700))
    k = int(rng.choice([4, 12, 30, 64, 100, 128, 256]))
    h, d = int(rng.choice([1, 2, 3, 4, 8, 16])), int(rng.choice([1, 4, 5, 8, 16, 20, 32]))
    bf16, masked = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    sys.stderr.write(f"[gpu] random value projection seed={seed} b={b} s={s} k={k} h={h} d={d} bf16={bf16} masked={masked}\n")
    sys.stderr.flush()
    x = rng.standard_normal((b, s, k)).astype(np.float32)
    w = (rng.standard_normal((h * d, k)) / np.sqrt(k)).astype(np.float32)
    bias = rng.standard_normal(h * d).astype(np.float32)
    mask = (rng.uniform(0, 1, (b, s)) < 0.2) if masked else None
    g = rng.standard_normal((b * h, s, d)).astype(np.float32)
    if bf16:
        x, g = bf16_round(x), bf16_round(g)
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32

    def t(a, dtype=torch.float32):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)

    tm = None if mask is None else torch.from_numpy(mask).to(dev)
    out = value_proj_forward(t(x, dt), t(w), t(bias), h, tm)
    gx, gw, gb = value_proj_backward(t(x, dt), t(w), h, t(g, dt), tm)
    torch.cuda.synchronize()
    wq = bf16_round(w) if bf16 else w  # the product sees weight.astype(x.dtype)
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out.float().cpu().numpy(), VP.value_proj_rows(x, wq, bias, h, mask), tf, "value")
    rx, rw, rb = VP.value_proj_rows_vjp(x, wq, h, g, mask)
    assert_close(gx.float().cpu().numpy(), rx, tg, "grad_input")
    assert_close(gw.float().cpu().numpy(), rw, tg, "grad_weight")
    assert_close(gb.float().cpu().numpy(), rb, tg, "grad_bias")


@pytest.mark.parametrize("seed", range(12))
def test_random_shape_grid_sample(seed):
    """The border/zeros grid sampler (msda_grid_sample_fwd / _bwd) on random [N, C, H, W] maps (up
    to 200 x 200, so some planes exceed the LDS budget and run in row bands) and grids reaching
    outside [-1, 1], f32 or bf16, against oracle/grid_sample_ref.py."""
    from oracle import grid_sample_ref as GS
    from oracle.msda_ref import bf16_round
    from rfdetr_jax_amd import grid_sample as gsm

    rng = np.random.default_rng(400 + seed)
    n, c = int(rng.integers(1, 5)), int(rng.choice([1, 2, 3, 4, 8, 16]))
    hh, ww = int(rng.integers(1, 201)), int(rng.integers(1, 201))
    gh, gw = int(rng.integers(1, 60)), int(rng.integers(1, 8))
    mode = "border" if rng.integers(0, 2) else "zeros"
    bf16 = bool(rng.integers(0, 2))
    sys.stderr.write(f"[gpu] random grid sample seed={seed} n={n} c={c} {hh}x{ww} grid {gh}x{gw} {mode} bf16={bf16}\n")
    sys.stderr.flush()
    inputs = rng.standard_normal((n, c, hh, ww)).astype(np.float32)
    grid = rng.uniform(-1.3, 1.3, (n, gh, gw, 2)).astype(np.float32)
    grad = rng.standard_normal((n, c, gh, gw)).astype(np.float32)
    if bf16:
        inputs, grad = bf16_round(inputs), bf16_round(grad)
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32
    ti = torch.from_numpy(inputs).to(dev).to(dt).requires_grad_(True)
    tgr = torch.from_numpy(grid).to(dev).requires_grad_(True)
    out = gsm.bilinear_grid_sample(ti, tgr, mode)
    out.backward(torch.from_numpy(grad).to(dev).to(dt))
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(out.float().detach().cpu().numpy(), GS.bilinear_grid_sample(inputs, grid, mode), tf, "out")
    gi, gg = GS.grid_sample_vjp(inputs, grid, grad, mode)
    assert_close(ti.grad.float().cpu().numpy(), gi, tg, "grad_input")
    assert_close(tgr.grad.cpu().numpy(), gg, tg, "grad_grid")


@pytest.mark.parametrize("seed", range(16))
def test_random_shape_attention(seed):
    """The decoder self-attention (msda_attention_fwd / _bwd and the dropout entry points) on random
    draws: [B, H, L, D] heads or [B, G * P, C] rows with G groups, L 1-400, head_dim 32 or 64, a
    key mask (with a fully blocked row) or none, dropout 0 or 0.15, f32 or bf16, against the
    float64 oracle given the kernels' keep mask. Whichever kernels the shape gets run: the fused
    or two-kernel backward, the staged or chunked bf16 forward."""
    from oracle import attention_ref as AT
    from oracle.msda_ref import bf16_round
    from rfdetr_jax_amd.attention import dropout_keep_mask, grouped_attention, scaled_dot_product_attention

    rng = np.random.default_rng(500 + seed)
    b, g_, h = int(rng.integers(1, 4)), int(rng.integers(1, 4)), int(rng.choice([1, 2, 4, 8]))
    length, d = int(rng.integers(1, 401)), int(rng.choice([32, 64]))
    rows, masked, bf16 = bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    rate = 0.15 if rng.integers(0, 2) else 0.0
    if not rows:
        g_ = 1
    sys.stderr.write(f"[gpu] random attention seed={seed} b={b} g={g_} h={h} L={length} d={d} rows={rows} masked={masked} "
                     f"bf16={bf16} dropout={rate}\n")
    sys.stderr.flush()
    z = g_ * b
    q, k, v, gr = (rng.standard_normal((z, h, length, d)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, gr = (bf16_round(x) for x in (q, k, v, gr))
    mask = None
    if masked:
        mask = rng.uniform(0, 1, (length, length)) < 0.2
        mask[length // 2] = True
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32
    seed_drop = 900 + seed

    def rows_of(x):  # [G B, H, L, D] -> [B, G L, H D] (slice z = g B + b)
        return x.reshape(g_, b, h, length, d).transpose(1, 0, 3, 2, 4).reshape(b, g_ * length, h * d)

    def heads_of(x):  # the inverse
        return x.reshape(b, g_, length, h, d).transpose(1, 0, 3, 2, 4).reshape(z, h, length, d)

    tm = None if mask is None else torch.from_numpy(mask).to(dev)
    if rows:
        tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(rows_of(x))).to(dev).to(dt).requires_grad_(True) for x in (q, k, v))
        out = grouped_attention(tq, tk, tv, h, g_, tm, dropout=rate, seed=seed_drop)
        out.backward(torch.from_numpy(np.ascontiguousarray(rows_of(gr))).to(dev).to(dt))
        got = [heads_of(t.detach().float().cpu().numpy()) for t in (out, tq.grad, tk.grad, tv.grad)]
    else:
        tq, tk, tv = (torch.from_numpy(x).to(dev).to(dt).requires_grad_(True) for x in (q, k, v))
        out = scaled_dot_product_attention(tq, tk, tv, tm, dropout=rate, seed=seed_drop)
        out.backward(torch.from_numpy(gr).to(dev).to(dt))
        got = [t.detach().float().cpu().numpy() for t in (out, tq.grad, tk.grad, tv.grad)]
    keep = None
    if rate > 0:
        keep = dropout_keep_mask(b, h, length, rate, seed_drop, groups=g_, device=dev).cpu().numpy().astype(bool)
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(got[0], AT.sdpa(q, k, v, mask, keep, rate), tf, "out")
    for name, mine, want in zip(("grad_q", "grad_k", "grad_v"), got[1:], AT.sdpa_vjp(q, k, v, gr, mask, keep, rate)):
        assert_close(mine, want, tg, name)


def _draw_wide(seed):
    """Many levels and points: 5-16 levels of 1-16 rows and columns, 1-40 points (up to 640
    samples per (query, head)), small heads and head_dim, so the oracle stays fast."""
    rng = np.random.default_rng(8000 + seed)
    levels = int(rng.integers(5, 17))
    shapes = tuple((int(rng.integers(1, 17)), int(rng.integers(1, 17))) for _ in range(levels))
    return dict(shapes=shapes, heads=int(rng.choice([1, 2, 3, 4])), dim=int(rng.choice([1, 2, 4, 8, 16])),
                points=int(rng.integers(1, 41)), queries=int(rng.integers(1, 101)), batch=int(rng.integers(1, 3)),
                bf16=bool(rng.integers(0, 2)), uniform=bool(rng.integers(0, 2)))


@pytest.mark.parametrize("seed", range(8))
def test_random_wide_shape_against_oracle(seed):
    """msda_fwd / msda_bwd, and the fused-prologue op (per-row prologue and epilogue kernels),
    with many levels and points against the float64 oracles."""
    from oracle import prologue_ref as PR
    from rfdetr_jax_amd.workloads import make_fused_inputs

    c = _draw_wide(seed)
    sys.stderr.write(f"[gpu] random wide shape seed={seed} {c}\n")
    sys.stderr.flush()
    dev = torch.device("cuda:0")
    tf, tg = (2e-2, 2e-2) if c["bf16"] else (1e-5, 1e-4)
    value, loc, attn, grad = make_inputs(800 + seed, c["batch"], c["heads"], c["dim"], c["queries"], c["shapes"], c["points"],
                                         value_dtype="bf16" if c["bf16"] else "f32", uniform_locations=c["uniform"])
    v = torch.from_numpy(value).to(dev)
    if c["bf16"]:
        v = v.to(torch.bfloat16)
    lc, a, g = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (loc, attn, grad))
    out = hip.ms_deform_attn_forward(v, c["shapes"], lc, a)
    gv, gl, ga = hip.ms_deform_attn_backward(v, c["shapes"], lc, a, g)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), R.ms_deform_attn_core_rows(value, c["shapes"], loc, attn), tf, "out")
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, c["shapes"], loc, attn, grad)
    assert_close(gv.float().cpu().numpy(), rv, tg, "grad_value")
    assert_close(gl.cpu().numpy(), rl, tg, "grad_loc")
    assert_close(ga.cpu().numpy(), ra, tg, "grad_attn")
    ref_dim = 2 if seed % 2 == 0 else 4
    value, ref, off, logits, grad = make_fused_inputs(900 + seed, c["batch"], c["heads"], c["dim"], c["queries"], c["shapes"],
                                                      c["points"], ref_dim, "bf16" if c["bf16"] else "f32")
    v = torch.from_numpy(value).to(dev)
    if c["bf16"]:
        v = v.to(torch.bfloat16)
    r, o, lg, g = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (ref, off, logits, grad))
    out = hip.ms_deform_attn_fused_forward(v, c["shapes"], r, o, lg)
    gv, gref, goff, glog = hip.ms_deform_attn_fused_backward(v, c["shapes"], r, o, lg, g)
    torch.cuda.synchronize()
    loc, attn = PR.prologue(ref, off, logits, c["shapes"], c["points"])
    rv, rl, ra = R.ms_deform_attn_core_rows_vjp(value, c["shapes"], loc, attn, grad)
    roff, rlog, rref = PR.prologue_vjp(ref, off, logits, c["shapes"], c["points"], rl, ra)
    assert_close(out.float().cpu().numpy(), R.ms_deform_attn_core_rows(value, c["shapes"], loc, attn), tf, "fused out")
    assert_close(gv.float().cpu().numpy(), rv, tg, "fused grad_value")
    assert_close(gref.cpu().numpy(), rref, tg, "grad_reference_points")
    assert_close(goff.cpu().numpy(), roff, tg, "grad_sampling_offsets")
    assert_close(glog.cpu().numpy(), rlog, tg, "grad_attention_logits")


@pytest.mark.parametrize("seed", range(8))
def test_random_shape_point_sample(seed):
    """point_sample (unit-square points, bilinear or nearest with border padding) on random maps
    and point layouts (flat [N, P, 2] or gridded [N, Hg, Wg, 2]), f32 or bf16, against the oracle
    (oracle/grid_sample_ref.py point_sample and its VJP)."""
    from oracle import grid_sample_ref as GS
    from oracle.msda_ref import bf16_round
    from rfdetr_jax_amd import grid_sample as gsm

    rng = np.random.default_rng(1400 + seed)
    n, c = int(rng.integers(1, 6)), int(rng.choice([1, 2, 3, 8]))
    hh, ww = int(rng.integers(1, 120)), int(rng.integers(1, 120))
    mode = "nearest" if rng.integers(0, 2) else "bilinear"
    bf16 = bool(rng.integers(0, 2))
    pts_shape = (n, int(rng.integers(1, 300)), 2) if rng.integers(0, 2) else (n, int(rng.integers(1, 20)), int(rng.integers(1, 20)), 2)
    sys.stderr.write(f"[gpu] random point sample seed={seed} n={n} c={c} {hh}x{ww} points {pts_shape} {mode} bf16={bf16}\n")
    sys.stderr.flush()
    inputs = rng.standard_normal((n, c, hh, ww)).astype(np.float32)
    pts = rng.uniform(-0.1, 1.1, pts_shape).astype(np.float32)
    grad = rng.standard_normal((n, c) + pts_shape[1:-1]).astype(np.float32)
    if bf16:
        inputs, grad = bf16_round(inputs), bf16_round(grad)
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if bf16 else torch.float32
    ti = torch.from_numpy(inputs).to(dev).to(dt).requires_grad_(True)
    tp = torch.from_numpy(pts).to(dev).requires_grad_(True)
    out = gsm.point_sample(ti, tp, mode)
    out.backward(torch.from_numpy(grad).to(dev).to(dt))
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    want = GS.point_sample(inputs, pts, mode)
    gi, gp = GS.point_sample_vjp(inputs, pts, grad, mode)
    assert_close(out.float().detach().cpu().numpy(), want, tf, "out")
    assert_close(ti.grad.float().cpu().numpy(), gi, tg, "grad_input")
    assert_close(tp.grad.cpu().numpy(), gp, tg, "grad_points")
