"""Pin the CPU oracles (oracle/msda_ref.py, oracle/msda_ref.c) before trusting them.

Checks, none of which retypes the oracle's formulas:
* the reference's closed-form known answers (tests/test_ops.py:22-54);
* torch ``F.grid_sample`` (bilinear, zeros, align_corners=False) — the routine ops.py:14-16 says
  the reference sampler reproduces — and torch autograd through it, in float64;
* central finite differences of the float64 forward;
* exact identities: the output is linear in value and in the weights, so
  ``<G, out> = <grad_value, value> = <grad_weights, weights>``;
* a pure-Python brute-force loop on tiny inputs;
* the C restatement against the NumPy one (forward and all gradients);
* the committed golden fixtures are reproduced.
Planted mistakes (a dropped corner, a transposed x/y, a wrong chain factor) are shown to fail.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import cref
from oracle import msda_ref as R
from rfdetr_jax_amd.workloads import make_inputs
from tests._util import assert_close, golden_names, load_golden


def _torch_reference(value, shapes, loc, attn, grad):
    from tests.golden.make_golden import torch_reference

    return torch_reference(value, shapes, loc, attn, grad)


# --------------------------------------------------------------------------------------------
# known answers of the reference's own tests


def test_kat_pixel_centres():
    """tests/test_ops.py:22-29: grid (-0.5,-0.5) -> 1, (0.5,0.5) -> 4 on [[1,2],[3,4]]."""
    value = np.array([1, 2, 3, 4], np.float32).reshape(1, 4, 1)
    loc = np.array([[0.25, 0.25], [0.75, 0.75]], np.float32).reshape(1, 2, 1, 1, 1, 2)
    out = R.ms_deform_attn_core_rows(value, ((2, 2),), loc, np.ones((1, 2, 1, 1), np.float32))
    assert out[0, 0, 0] == pytest.approx(1.0) and out[0, 1, 0] == pytest.approx(4.0)
    assert cref.forward(value, ((2, 2),), loc, np.ones((1, 2, 1, 1), np.float32))[0, :, 0] == pytest.approx([1.0, 4.0])


def test_kat_zero_pad():
    """tests/test_ops.py:32-36: a sample far outside contributes exactly 0."""
    out = R.ms_deform_attn_core_rows(np.ones((1, 4, 1), np.float32), ((2, 2),),
                                     np.full((1, 1, 1, 1, 1, 2), 3.0, np.float32), np.ones((1, 1, 1, 1), np.float32))
    assert out[0, 0, 0] == 0.0


def test_kat_midpoint():
    """tests/test_ops.py:39-43: midway between pixel values 0 and 4 gives 2."""
    out = R.ms_deform_attn_core_rows(np.array([0, 4], np.float32).reshape(1, 2, 1), ((1, 2),),
                                     np.full((1, 1, 1, 1, 1, 2), 0.5, np.float32), np.ones((1, 1, 1, 1), np.float32))
    assert out[0, 0, 0] == pytest.approx(2.0)


def test_kat_mean_of_points():
    """tests/test_ops.py:46-54: uniform weights over two points of arange(4) give 1.5."""
    out = R.ms_deform_attn_core_rows(np.arange(4, dtype=np.float32).reshape(1, 4, 1), ((2, 2),),
                                     np.array([[0.25, 0.25], [0.75, 0.75]], np.float32).reshape(1, 1, 1, 1, 2, 2),
                                     np.full((1, 1, 1, 2), 0.5, np.float32))
    assert out.shape == (1, 1, 1)
    assert out[0, 0, 0] == pytest.approx(1.5)


# --------------------------------------------------------------------------------------------
# independent references


def _random_case(seed, shapes=((8, 16), (4, 8)), b=2, q=23, h=2, p=3, d=8, lo=-0.2, hi=1.2, dtype=np.float32):
    rng = np.random.default_rng(seed)
    s = sum(x * y for x, y in shapes)
    value = rng.standard_normal((b * h, s, d)).astype(dtype)
    loc = rng.uniform(lo, hi, (b, q, h, len(shapes), p, 2)).astype(dtype)
    attn = rng.uniform(0, 1, (b, q, h, len(shapes) * p)).astype(dtype)
    grad = rng.standard_normal((b, q, h * d)).astype(dtype)
    return value, loc, attn, grad


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_forward_matches_torch_grid_sample(seed):
    value, loc, attn, grad = _random_case(seed)
    shapes = ((8, 16), (4, 8))
    want = _torch_reference(value, shapes, loc, attn, grad)[0]
    assert_close(R.ms_deform_attn_core_rows(value, shapes, loc, attn), want, 1e-6, "forward vs grid_sample")


@pytest.mark.parametrize("seed", [0, 1])
def test_vjp_matches_torch_autograd_float64(seed):
    """float64 inputs: coordinates are float64 too (ops.py:269-270), as in torch."""
    shapes = ((8, 16), (4, 8))
    value, loc, attn, grad = _random_case(seed, dtype=np.float64)
    _, t_gv, t_gl, t_ga = _torch_reference(value, shapes, loc, attn, grad)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(gv, t_gv, 1e-12, "grad_value")
    assert_close(gl, t_gl, 1e-12, "grad_loc")
    assert_close(ga, t_ga, 1e-12, "grad_attn")


def test_vjp_matches_finite_differences():
    shapes = ((6, 7), (3, 4))
    value, loc, attn, grad = _random_case(5, shapes=shapes, b=1, q=5, h=2, p=2, d=3, lo=0.05, hi=0.95, dtype=np.float64)
    # Keep every sample away from pixel-cell boundaries, where floor() makes the map kinked.
    for lvl, (hl, wl) in enumerate(shapes):
        for axis, size in ((0, wl), (1, hl)):
            pix = loc[:, :, :, lvl, :, axis] * size - 0.5
            frac = pix - np.floor(pix)
            pix = np.where(frac < 0.05, pix + 0.1, np.where(frac > 0.95, pix - 0.1, pix))
            loc[:, :, :, lvl, :, axis] = (pix + 0.5) / size
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)

    def f(v, lc, a):
        return float(np.sum(R.ms_deform_attn_core_rows(v, shapes, lc, a) * grad))

    eps = 1e-6
    rng = np.random.default_rng(0)
    for name, arr, analytic in (("value", value, gv), ("loc", loc, gl), ("attn", attn, ga)):
        flat_idx = rng.choice(arr.size, size=min(25, arr.size), replace=False)
        for i in flat_idx:
            plus, minus = arr.copy(), arr.copy()
            plus.reshape(-1)[i] += eps
            minus.reshape(-1)[i] -= eps
            args_p = {"value": (plus, loc, attn), "loc": (value, plus, attn), "attn": (value, loc, plus)}[name]
            args_m = {"value": (minus, loc, attn), "loc": (value, minus, attn), "attn": (value, loc, minus)}[name]
            numeric = (f(*args_p) - f(*args_m)) / (2 * eps)
            assert abs(numeric - analytic.reshape(-1)[i]) <= 1e-6 * max(1.0, abs(numeric)), (name, i)


def test_linearity_identities():
    """out is linear in value and in weights: <G,out> = <dV,V> = <dA,A> exactly (up to rounding)."""
    shapes = ((8, 16), (4, 8))
    value, loc, attn, grad = _random_case(9)
    out = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    gv, _, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    inner = float(np.sum(out * grad))
    assert np.sum(gv * value) == pytest.approx(inner, rel=1e-10, abs=1e-10)
    assert np.sum(ga * attn) == pytest.approx(inner, rel=1e-10, abs=1e-10)


def test_brute_force_loop_agrees():
    shapes = ((5, 4), (2, 3))
    value, loc, attn, _ = _random_case(4, shapes=shapes, b=2, q=3, h=2, p=2, d=3)
    assert_close(R.ms_deform_attn_core_rows(value, shapes, loc, attn),
                 R.brute_force_forward(value, shapes, loc, attn), 1e-12, "brute force")


def test_integer_translation():
    """Shifting every sample by exactly one pixel to the right equals sampling a map shifted left."""
    shapes = ((8, 16),)
    rng = np.random.default_rng(12)
    value = rng.standard_normal((2, 128, 4)).astype(np.float32)
    # dyadic locations keep every coordinate exact in f32
    loc = (rng.integers(8, 120, (1, 9, 2, 1, 2, 2)) / 128.0).astype(np.float32)
    attn = rng.uniform(0, 1, (1, 9, 2, 2)).astype(np.float32)
    moved = loc.copy()
    moved[..., 0] += np.float32(1.0 / 16)
    shifted = np.zeros_like(value).reshape(2, 8, 16, 4)
    shifted[:, :, :-1] = value.reshape(2, 8, 16, 4)[:, :, 1:]
    a = R.ms_deform_attn_core_rows(value, shapes, moved, attn)
    b = R.ms_deform_attn_core_rows(shifted.reshape(2, 128, 4), shapes, loc, attn)
    assert_close(a, b, 1e-12, "translation")


# --------------------------------------------------------------------------------------------
# planted mistakes must be caught by the references above


def test_planted_mistakes_are_caught(monkeypatch):
    shapes = ((8, 16), (4, 8))
    value, loc, attn, grad = _random_case(1)
    want = _torch_reference(value, shapes, loc, attn, grad)
    orig = R._corners

    def dropped_corner(*a):
        idx, w, m, fx, fy = orig(*a)
        w = w.copy()
        w[..., 3] = 0.0
        return idx, w, m, fx, fy

    def swapped_xy(loc_x, loc_y, height, width):
        return orig(loc_y, loc_x, height, width)

    for bad in (dropped_corner, swapped_xy):
        monkeypatch.setattr(R, "_corners", bad)
        with pytest.raises(AssertionError):
            assert_close(R.ms_deform_attn_core_rows(value, shapes, loc, attn), want[0], 1e-6, bad.__name__)
        monkeypatch.setattr(R, "_corners", orig)
    # a wrong chain factor (d ix/d loc = W/2 instead of W) shows up in grad_loc only
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    with pytest.raises(AssertionError):
        assert_close(gl / 2, want[2], 1e-6, "half chain factor")


# --------------------------------------------------------------------------------------------
# the C restatement (used as full-size oracle and CPU baseline)


@pytest.mark.parametrize("seed", [0, 3])
def test_c_oracle_matches_numpy(seed):
    shapes = ((8, 16), (4, 8))
    value, loc, attn, grad = _random_case(seed, q=31)
    assert_close(cref.forward(value, shapes, loc, attn), R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-6, "fwd")
    cv, cl, ca = cref.backward(value, shapes, loc, attn, grad)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(cv, gv, 1e-6, "grad_value")
    assert_close(cl, gl, 1e-5, "grad_loc")
    assert_close(ca, ga, 1e-6, "grad_attn")


def test_c_oracle_config1_size():
    """Benchmark config 1 at full size (B=16, 24x24, Q=300, P=2): C vs NumPy oracle."""
    value, loc, attn, grad = make_inputs(1, 16, 16, 16, 300, ((24, 24),), 2)
    shapes = ((24, 24),)
    assert_close(cref.forward(value, shapes, loc, attn), R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "fwd")
    cv, cl, ca = cref.backward(value, shapes, loc, attn, grad)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(value, shapes, loc, attn, grad)
    assert_close(cv, gv, 1e-5, "grad_value")
    assert_close(cl, gl, 1e-4, "grad_loc")
    assert_close(ca, ga, 1e-5, "grad_attn")


# --------------------------------------------------------------------------------------------
# golden fixtures


@pytest.mark.parametrize("name", golden_names())
def test_golden_fixture_reproduced(name):
    g = load_golden(name)
    out = R.ms_deform_attn_core_rows(g["value"], g["shapes"], g["loc"], g["attn"])
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp(g["value"], g["shapes"], g["loc"], g["attn"], g["grad"])
    assert_close(out, g["out"], 1e-6, "out")
    assert_close(gv, g["grad_value"], 1e-6, "grad_value")
    assert_close(gl, g["grad_loc"], 1e-6, "grad_loc")
    assert_close(ga, g["grad_attn"], 1e-6, "grad_attn")
    if "expect" in g["meta"]:
        assert np.allclose(out.reshape(-1), g["meta"]["expect"])


def test_bf16_round():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, np.inf], np.float32)
    r = R.bf16_round(x)
    assert r[0] == 1.0 and r[1] == 1.0  # tie -> even
    assert r[2] == np.float32(1.0078125)
    assert r[3] == -2.5 and np.isinf(r[5])
    assert np.isnan(R.bf16_round(np.array([np.nan], np.float32))[0])


def test_bf16_gather_emulation_exact_where_bf16_is_exact():
    """The emulation of the reference's bf16 rounding points (ops.py:88-91, :123-134) equals the
    float64 forward when every rounding it applies is exact: quarter-pixel positions on 8-wide and
    4-high levels (fractions and weight products are multiples of 1/16), integer values in [-2, 2]
    (corner products and four-corner sums need at most 6 significant bits)."""
    rng = np.random.default_rng(11)
    shapes = ((8, 8), (4, 8))
    b, q, h, d, p = 2, 9, 2, 4, 3
    s = sum(hh * ww for hh, ww in shapes)
    value = rng.integers(-2, 3, size=(b * h, s, d)).astype(np.float32)
    loc = np.empty((b, q, h, len(shapes), p, 2), np.float32)
    for lvl, (hh, ww) in enumerate(shapes):
        # ix = loc * W - 0.5 in quarter pixels from -1.5 to W + 0.5 (edges and outside included)
        ix = rng.integers(-6, 4 * ww + 3, size=(b, q, h, p)) / 4.0
        iy = rng.integers(-6, 4 * hh + 3, size=(b, q, h, p)) / 4.0
        loc[:, :, :, lvl, :, 0] = (ix + 0.5) / ww
        loc[:, :, :, lvl, :, 1] = (iy + 0.5) / hh
    attn = rng.random((b, q, h, len(shapes) * p)).astype(np.float32)
    want = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    got = R.ms_deform_attn_core_rows_bf16_gather(value, shapes, loc, attn)
    np.testing.assert_array_equal(got, want)


def test_bf16_gather_emulation_planted_mistake_and_gap():
    """Rounding the coordinate instead of its fraction (a plausible misreading of ops.py:88) changes
    the result on an 80-wide level; and the emulated reference stays within the bf16 parity
    tolerance (2e-2) of the f32 interpolation the kernels compute, at the two-level shape."""
    shapes = ((80, 80), (20, 20))
    value, loc, attn, _ = make_inputs(3, 1, 4, 16, 120, shapes, 4)
    value = R.bf16_round(value)
    emu = R.ms_deform_attn_core_rows_bf16_gather(value, shapes, loc, attn)
    planted = R.ms_deform_attn_core_rows_bf16_gather(value, shapes, loc, attn, _round_coordinate=True)
    assert np.abs(planted - emu).max() > 1e-2
    f32_path = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    gap = np.abs(emu - f32_path).max() / max(1.0, np.abs(f32_path).max())
    assert 1e-4 < gap < 2e-2, gap


# --------------------------------------------------------------------------------------------
# the samplers' rounding points (ms_deform_attn_core_rows_sampler)


def _torch_bf16_sampler_level(value_l, loc, height, width, mode):
    """The reference's per-level samplers written with torch tensors of the dtypes the reference
    uses (ops.py:64-186): every bf16 operation rounds by itself, as XLA's bf16 arithmetic does, so
    where the oracle places its explicit bf16 roundings is checked against arithmetic that rounds
    at every step. value_l [N, S, D] bf16-representable float32; loc [N, L, 2]. Returns [N, L, D]."""
    import torch

    bf = torch.bfloat16
    v = torch.from_numpy(value_l).to(bf)
    g = 2 * torch.from_numpy(loc).float() - 1
    ix = ((g[..., 0] + 1) * width - 1) / 2
    iy = ((g[..., 1] + 1) * height - 1) / 2
    ix0, iy0 = torch.floor(ix), torch.floor(iy)
    if mode == "matmul":
        wx1, wy1 = (ix - ix0)[..., None], (iy - iy0)[..., None]
        cols = torch.arange(width, dtype=torch.float32)
        rows = torch.arange(height, dtype=torch.float32)
        kx = torch.where(cols == ix0[..., None], 1 - wx1, 0.0) + torch.where(cols == ix0[..., None] + 1, wx1, 0.0)
        ky = torch.where(rows == iy0[..., None], 1 - wy1, 0.0) + torch.where(rows == iy0[..., None] + 1, wy1, 0.0)
        kernel = (ky.to(bf)[..., :, None] * kx.to(bf)[..., None, :]).reshape(*loc.shape[:2], height * width)
        return torch.bmm(kernel.float(), v.float()).to(bf).float().numpy()  # f32 contraction, bf16 result
    dt = bf if mode == "gather" else torch.float32
    vv = v.to(dt)
    wx1, wy1 = (ix - ix0).to(dt)[..., None], (iy - iy0).to(dt)[..., None]
    wx0, wy0 = 1 - wx1, 1 - wy1
    x0, y0 = ix0.long(), iy0.long()
    x1, y1 = x0 + 1, y0 + 1
    ins = [((xx >= 0) & (xx < width) & (yy >= 0) & (yy < height)) for xx, yy in ((x0, y0), (x1, y0), (x0, y1), (x1, y1))]
    idx = [yy.clamp(0, height - 1) * width + xx.clamp(0, width - 1) for xx, yy in ((x0, y0), (x1, y0), (x0, y1), (x1, y1))]
    weights = [wx0 * wy0, wx1 * wy0, wx0 * wy1, wx1 * wy1]
    prods = []
    for c in range(4):
        corner = torch.gather(vv, 1, idx[c][..., None].expand(-1, -1, vv.shape[-1]))
        prods.append(corner * (weights[c] * ins[c][..., None].to(dt)))
    total = torch.stack(prods, 1).float().sum(1)  # the four-corner sum in f32
    return total.to(bf).float().numpy()


@pytest.mark.parametrize("mode", ["gather", "gather-f32", "matmul"])
def test_bf16_sampler_rounding_points_match_rounding_arithmetic(mode):
    """The oracle's explicit bf16 roundings of each sampler equal torch arithmetic in the dtypes the
    reference computes in (bf16 ops round after every operation): a missing or extra rounding
    point changes some of the 1920 samples."""
    rng = np.random.default_rng(5)
    shapes = ((13, 17),)
    n, q, p, d = 4, 60, 2, 8
    value = R.bf16_round(rng.standard_normal((n, 13 * 17, d)).astype(np.float32))
    loc = rng.uniform(-0.1, 1.1, (n, q * p, 2)).astype(np.float32)
    want = _torch_bf16_sampler_level(value, loc, 13, 17, mode)
    got = R._bf16_level_sample(value.reshape(1, n, -1, d), loc.reshape(1, q, n, p, 2).transpose(0, 1, 2, 3, 4).reshape(1, n, q, p, 2).transpose(0, 2, 1, 3, 4), 13, 17, mode)
    got = got.transpose(0, 2, 1, 3, 4).reshape(n, q * p, d)
    np.testing.assert_array_equal(got, want)


def test_sampler_emulations_exact_where_bf16_is_exact():
    """Every sampler's emulation equals the float64 forward when each rounding it applies is exact:
    quarter-pixel positions on power-of-two levels (both pixel-coordinate formulas exact; fractions
    and weight products multiples of 1/16), integer values in [-2, 2]."""
    rng = np.random.default_rng(12)
    shapes = ((8, 8), (4, 8))
    b, q, h, d, p = 2, 9, 2, 4, 3
    s = sum(hh * ww for hh, ww in shapes)
    value = rng.integers(-2, 3, size=(b * h, s, d)).astype(np.float32)
    loc = np.empty((b, q, h, len(shapes), p, 2), np.float32)
    for lvl, (hh, ww) in enumerate(shapes):
        loc[:, :, :, lvl, :, 0] = (rng.integers(-6, 4 * ww + 3, size=(b, q, h, p)) / 4.0 + 0.5) / ww
        loc[:, :, :, lvl, :, 1] = (rng.integers(-6, 4 * hh + 3, size=(b, q, h, p)) / 4.0 + 0.5) / hh
    attn = rng.random((b, q, h, len(shapes) * p)).astype(np.float32)
    want = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    for sampler in ("gather", "gather-f32", "matmul", "auto", "pallas"):
        for bf in (True, False):
            got = R.ms_deform_attn_core_rows_sampler(value, shapes, loc, attn, sampler, bf)
            np.testing.assert_array_equal(got, want, err_msg=f"{sampler} bf16={bf}")


def test_pallas_pixel_coordinates():
    """The Pallas sampler's coordinates are loc * size - 0.5 in float32 (two roundings, torch f32
    arithmetic as the checker); at an 80-wide level they differ from ops.py's
    ((2 loc - 1 + 1) size - 1) / 2 for some positions, and where a floor decision differs the
    sampler's output does."""
    import torch

    # positions within a few ulps of the cell boundaries (k + 1/2) / 80, where a floor can flip
    edges = ((np.arange(-1, 81) + 0.5) / 80).astype(np.float32)
    steps = np.arange(-8, 9)
    loc = np.array([np.nextafter(e, np.float32(2 if k > 0 else -1)) if k else e for e in edges for k in steps], np.float32)
    for _ in range(7):  # widen to +-8 ulps
        loc = np.concatenate([loc, np.nextafter(loc, np.float32(2)), np.nextafter(loc, np.float32(-1))])
    want = (torch.from_numpy(loc) * 80.0 - 0.5).numpy()
    np.testing.assert_array_equal(R._pallas_coords(loc, 80), want)
    gather_xy = R._pixel_coords(loc, 80).astype(np.float32)
    differ = np.floor(want) != np.floor(gather_xy)
    assert differ.any() and (want != gather_xy).mean() > 0.01
    # one sample at a position whose floor differs: the two samplers read different cells
    inner = differ & (np.floor(want) >= 1) & (np.floor(want) <= 77)
    assert inner.any()
    x = loc[np.argmax(inner)]
    value = np.arange(80 * 2, dtype=np.float32).reshape(1, 160, 1)
    sl = np.array([x, 0.25], np.float32).reshape(1, 1, 1, 1, 1, 2)
    a = np.ones((1, 1, 1, 1), np.float32)
    out_p = R.ms_deform_attn_core_rows_sampler(value, ((2, 80),), sl, a, "pallas", False)
    out_g = R.ms_deform_attn_core_rows_sampler(value, ((2, 80),), sl, a, "gather", False)
    assert out_p[0, 0, 0] != out_g[0, 0, 0]


def test_pallas_vjp_is_the_vjp_at_pallas_coordinates():
    """ms_deform_attn_core_rows_vjp_pallas against central finite differences of the Pallas
    forward emulation (float64 interpolation) in the value and the weights, and the identity
    <G, out> = <dV, V> = <dA, A>."""
    shapes = ((5, 7), (3, 4))
    value, loc, attn, grad = make_inputs(21, 1, 2, 3, 6, shapes, 2)
    out = R.ms_deform_attn_core_rows_sampler(value, shapes, loc, attn, "pallas", False)
    gv, gl, ga = R.ms_deform_attn_core_rows_vjp_pallas(value, shapes, loc, attn, grad)
    g = grad.astype(np.float64)
    assert np.isclose((g * out).sum(), (gv * value).sum(), rtol=1e-10)
    assert np.isclose((g * out).sum(), (ga * attn).sum(), rtol=1e-10)
    eps = 1e-3
    for i in range(0, value.size, 7):
        vp = value.astype(np.float64).copy().reshape(-1)
        vm = vp.copy()
        vp[i] += eps
        vm[i] -= eps
        fp = R.ms_deform_attn_core_rows_sampler(vp.reshape(value.shape), shapes, loc, attn, "pallas", False)
        fm = R.ms_deform_attn_core_rows_sampler(vm.reshape(value.shape), shapes, loc, attn, "pallas", False)
        assert np.isclose((g * (fp - fm)).sum() / (2 * eps), gv.reshape(-1)[i], atol=1e-6)
