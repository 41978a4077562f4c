"""Pin the value-projection oracle (oracle/value_proj_ref.py) before trusting it.

Checks, none of which retypes the oracle's formulas: torch float64 ``F.linear`` + ``masked_fill``
+ ``view``/``permute`` under autograd (forward and the three gradients); closed forms (an identity
weight copies input channels into heads in order; padded rows are zero whatever the bias).
Planted mistakes (heads and positions swapped in the split, the mask applied before the bias) fail.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import value_proj_ref as VP
from tests._util import assert_close


def _case(seed, b=2, s=11, k=12, h=4, d=3, masked=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, s, k)).astype(np.float32)
    w = rng.standard_normal((h * d, k)).astype(np.float32)
    bias = rng.standard_normal(h * d).astype(np.float32)
    mask = (rng.uniform(0, 1, (b, s)) < 0.3) if masked else None
    g = rng.standard_normal((b * h, s, d)).astype(np.float32)
    return x, w, bias, mask, g, h


def _torch(x, w, bias, mask, g, h):
    import torch
    import torch.nn.functional as F

    tx = torch.tensor(x.astype(np.float64), requires_grad=True)
    tw = torch.tensor(w.astype(np.float64), requires_grad=True)
    tb = torch.tensor(bias.astype(np.float64), requires_grad=True)
    y = F.linear(tx, tw, tb)
    if mask is not None:
        y = y.masked_fill(torch.tensor(mask)[..., None], 0.0)
    b, s, n = y.shape
    v = y.view(b, s, h, n // h).permute(0, 2, 1, 3).reshape(b * h, s, n // h)
    v.backward(torch.tensor(g.astype(np.float64)))
    return v.detach().numpy(), tx.grad.numpy(), tw.grad.numpy(), tb.grad.numpy()


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("seed", [0, 1])
def test_matches_torch_autograd(seed, masked):
    x, w, bias, mask, g, h = _case(seed, masked=masked)
    tv, tgx, tgw, tgb = _torch(x, w, bias, mask, g, h)
    assert_close(VP.value_proj_rows(x, w, bias, h, mask), tv, 1e-12, "value")
    gx, gw, gb = VP.value_proj_rows_vjp(x, w, h, g, mask)
    assert_close(gx, tgx, 1e-12, "grad_x")
    assert_close(gw, tgw, 1e-12, "grad_w")
    assert_close(gb, tgb, 1e-12, "grad_b")


def _check_identity(fn):
    b, s, h, d = 2, 5, 3, 4
    x = np.arange(b * s * h * d, dtype=np.float32).reshape(b, s, h * d)
    v = fn(x, np.eye(h * d, dtype=np.float32), None, h, None)
    for bb in range(b):
        for hh in range(h):
            assert np.array_equal(v[bb * h + hh], x[bb, :, hh * d:(hh + 1) * d])


def _check_padded_rows_zero(fn):
    x, w, bias, mask, g, h = _case(3)
    v = fn(x, w, bias, h, mask)
    b, s = mask.shape
    vv = v.reshape(b, h, s, -1)
    assert np.all(vv[np.broadcast_to(mask[:, None, :], (b, h, s))] == 0.0)
    assert np.any(vv[np.broadcast_to(~mask[:, None, :], (b, h, s))] != 0.0)


@pytest.mark.parametrize("check", [_check_identity, _check_padded_rows_zero], ids=lambda c: c.__name__)
def test_closed_forms(check):
    check(VP.value_proj_rows)


def _swapped_split(x, w, bias, h, mask):
    v = VP.value_proj_rows(x, w, bias, h, mask)
    b, s = x.shape[:2]
    d = v.shape[-1]
    return v.reshape(b, h, s, d).transpose(0, 2, 1, 3).reshape(b * h, s, d) if s != h else v[::-1]


def _mask_before_bias(x, w, bias, h, mask):
    xm = x if mask is None else np.where(mask[..., None], 0.0, x)
    return VP.value_proj_rows(xm, w, bias, h, None)


@pytest.mark.parametrize("mistake", [_swapped_split, _mask_before_bias], ids=lambda m: m.__name__)
def test_planted_mistakes_are_caught(mistake):
    failed = 0
    for check in (_check_identity, _check_padded_rows_zero):
        try:
            check(mistake)
        except (AssertionError, ValueError):
            failed += 1
    assert failed > 0
