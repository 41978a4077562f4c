"""Pin the attention oracle (oracle/attention_ref.py) before trusting it.

Checks, none of which retypes the oracle's formulas: torch float64 ``F.scaled_dot_product_attention``
and ``nn.MultiheadAttention(batch_first=True)`` under autograd; the reference's own checks
(tests/test_attention.py: a masked key block; equal scores give the mean of V;
tests/test_transformer.py:20-38: group folding); closed forms; planted mistakes fail them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_ref as AT
from tests._util import assert_close


def _qkv(seed, shape=(2, 3, 9, 16)):
    rng = np.random.default_rng(seed)
    return tuple(rng.standard_normal(shape).astype(np.float32) for _ in range(3))


@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_matches_torch_autograd(masked):
    q, k, v = _qkv(1, (2, 3, 11, 8))
    mask = None
    if masked:
        mask = np.zeros((11, 11), bool)
        mask[:, -3:] = True  # tests/test_attention.py:37-40
        mask[2, :5] = True
    g = np.random.default_rng(2).standard_normal(q.shape)
    tq, tk, tv = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    out = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=None if mask is None else ~torch.tensor(mask))
    out.backward(torch.tensor(g))
    assert_close(AT.sdpa(q, k, v, mask), out.detach().numpy(), 1e-12, "out")
    for name, mine, want in zip("qkv", AT.sdpa_vjp(q, k, v, g, mask), (tq.grad, tk.grad, tv.grad)):
        assert_close(mine, want.numpy(), 1e-12, f"d{name}")


def test_reference_known_answers():
    q, k, v = _qkv(0)
    # tests/test_attention.py:14-21: blocked keys as -inf scores
    mask = np.zeros((9, 9), bool)
    mask[:, -3:] = True
    s = q.astype(np.float64) @ np.swapaxes(k, -1, -2) / np.sqrt(16)
    s = np.where(mask, -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    assert_close(AT.sdpa(q, k, v, mask), (e / e.sum(-1, keepdims=True)) @ v, 1e-12, "masked")
    # tests/test_attention.py:104-119: equal scores give the mean of V
    ones = np.ones((2, 3, 145, 16), np.float32)
    vv = np.random.default_rng(0).standard_normal((2, 3, 145, 16)).astype(np.float32)
    out = AT.sdpa(ones, -ones, vv)
    assert_close(out, np.broadcast_to(vv.astype(np.float64).mean(2, keepdims=True), out.shape), 1e-12, "mean")


def test_closed_forms():
    q, k, v = _qkv(3, (1, 2, 7, 4))
    # a fully blocked row: every score is finfo.min, so the weights are uniform (mean of V)
    mask = np.zeros((7, 7), bool)
    mask[4] = True
    out = AT.sdpa(q, k, v, mask)
    assert_close(out[:, :, 4], v.astype(np.float64).mean(2), 1e-12, "blocked row")
    # one dominant key selects its value row
    kk = np.zeros_like(k)
    kk[:, :, 5] = 60.0
    qq = np.ones_like(q)
    out = AT.sdpa(qq, kk, v)
    assert_close(out, np.broadcast_to(v[:, :, 5:6].astype(np.float64), out.shape), 1e-9, "one-hot")
    # the VJP of a linear functional: <grad, out(v)> is linear in v, so dv is P^T grad exactly
    g = np.random.default_rng(4).standard_normal(q.shape)
    _, _, dv = AT.sdpa_vjp(q, k, v, g)
    eps = 1e-6
    e = np.zeros_like(v, dtype=np.float64)
    e[0, 1, 3, 2] = eps
    num = ((AT.sdpa(q, k, v + e) - AT.sdpa(q, k, v)) * g).sum() / eps
    assert abs(num - dv[0, 1, 3, 2]) < 1e-6


def test_group_folding_matches_the_reference_ordering():
    """tests/test_transformer.py:20-38: round trip, and group g of image b lands at row g * B + b."""
    batch, groups, per = 2, 3, 4
    x = np.arange(batch * groups * per, dtype=np.float32).reshape(batch, groups * per, 1)
    folded = AT.split_groups(x, per)
    for g in range(groups):
        for b in range(batch):
            assert np.array_equal(folded[g * batch + b], x[b, g * per:(g + 1) * per])
    assert np.array_equal(AT.merge_groups(folded, batch), x)


def _torch_mha(params, query, key, value, heads, mask=None):
    c = query.shape[-1]
    m = torch.nn.MultiheadAttention(c, heads, batch_first=True, dtype=torch.float64)
    with torch.no_grad():
        m.in_proj_weight.copy_(torch.tensor(params["in_w"]))
        m.in_proj_bias.copy_(torch.tensor(params["in_b"]))
        m.out_proj.weight.copy_(torch.tensor(params["out_w"]))
        m.out_proj.bias.copy_(torch.tensor(params["out_b"]))
    t = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    out, _ = m(t(query), t(key), t(value), attn_mask=None if mask is None else torch.tensor(mask), need_weights=False)
    return out.detach().numpy()


def _params(seed, c):
    rng = np.random.default_rng(seed)
    return {"in_w": rng.standard_normal((3 * c, c)) / np.sqrt(c), "in_b": rng.standard_normal(3 * c) * 0.1,
            "out_w": rng.standard_normal((c, c)) / np.sqrt(c), "out_b": rng.standard_normal(c) * 0.1}


def test_multihead_attention_matches_torch():
    c, heads = 16, 4
    p = _params(5, c)
    rng = np.random.default_rng(6)
    query, key, value = (rng.standard_normal((2, 7, c)) for _ in range(3))
    mask = np.zeros((7, 7), bool)
    mask[:, 5:] = True
    for m in (None, mask):
        mine = AT.multihead_attention(query, key, value, p["in_w"], p["in_b"], p["out_w"], p["out_b"], heads, m)
        assert_close(mine, _torch_mha(p, query, key, value, heads, m), 1e-12, "mha")


def test_decoder_self_attention_is_mha_per_group():
    """Grouped self-attention equals running torch's MHA on each (image, group) block alone."""
    c, heads, batch, groups, per = 16, 4, 2, 3, 5
    p = _params(7, c)
    rng = np.random.default_rng(8)
    tgt = rng.standard_normal((batch, groups * per, c))
    pos = rng.standard_normal((batch, groups * per, c))
    mine = AT.decoder_self_attention(tgt, pos, groups, p["in_w"], p["in_b"], p["out_w"], p["out_b"], heads)
    for b in range(batch):
        for g in range(groups):
            sl = slice(g * per, (g + 1) * per)
            qk = (tgt + pos)[b:b + 1, sl]
            want = _torch_mha(p, qk, qk, tgt[b:b + 1, sl], heads)
            assert_close(mine[b:b + 1, sl], want, 1e-12, f"group {g} image {b}")


@pytest.mark.parametrize("mistake", ["no_scale", "softmax_over_queries", "image_major_folding"])
def test_planted_mistakes_are_caught(mistake, monkeypatch):
    q, k, v = _qkv(9, (1, 2, 6, 4))
    if mistake == "no_scale":
        def bad(q_, k_, mask):
            s = np.asarray(q_, np.float64) @ np.swapaxes(np.asarray(k_, np.float64), -1, -2)
            e = np.exp(s - s.max(-1, keepdims=True))
            return e / e.sum(-1, keepdims=True)
        monkeypatch.setattr(AT, "_probs", bad)
    elif mistake == "softmax_over_queries":
        def bad(q_, k_, mask):
            s = np.asarray(q_, np.float64) @ np.swapaxes(np.asarray(k_, np.float64), -1, -2) / np.sqrt(q_.shape[-1])
            e = np.exp(s - s.max(-2, keepdims=True))
            return e / e.sum(-2, keepdims=True)
        monkeypatch.setattr(AT, "_probs", bad)
    else:
        monkeypatch.setattr(AT, "split_groups", lambda x, per: np.asarray(x).reshape(-1, per, np.asarray(x).shape[-1]))
    with pytest.raises(AssertionError):
        if mistake == "image_major_folding":
            test_group_folding_matches_the_reference_ordering()
        else:
            tq, tk, tv = (torch.tensor(t, dtype=torch.float64) for t in (q, k, v))
            assert_close(AT.sdpa(q, k, v), F.scaled_dot_product_attention(tq, tk, tv).numpy(), 1e-9, "planted")


def test_fully_blocked_row_gradients_match_torch_masked_fill():
    """A row whose every key is blocked: the scores all become finfo(float32).min, the weights are
    uniform (the output is the mean of V), and ``where`` (torch's masked_fill here, jnp.where in
    layers.py:93-96) passes the blocked scores no gradient, so the row's dQ is 0 and it adds nothing
    to dK; dV still receives the uniform weights. torch float64 autograd."""
    q, k, v = _qkv(23, (2, 2, 9, 8))
    mask = np.zeros((9, 9), bool)
    mask[3] = True
    mask[:, 7] = True
    g = np.random.default_rng(6).standard_normal(q.shape)
    tq, tk, tv = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    scores = (tq @ tk.transpose(-1, -2) / np.sqrt(8)).masked_fill(torch.tensor(mask), float(np.finfo(np.float32).min))
    out = torch.softmax(scores, -1) @ tv
    out.backward(torch.tensor(g))
    assert_close(AT.sdpa(q, k, v, mask), out.detach().numpy(), 1e-12, "out")
    dq, dk, dv = AT.sdpa_vjp(q, k, v, g, mask)
    assert not dq[:, :, 3].any()
    for name, mine, want in zip("qkv", (dq, dk, dv), (tq.grad, tk.grad, tv.grad)):
        assert_close(mine, want.numpy(), 1e-12, f"d{name}")


def _torch_dropout_attention(q, k, v, mask, rate, seed):
    """torch float64: softmax attention whose weights go through ``F.dropout`` (training), the
    keep mask read back from which weights survived; returns (out, keep, autograd leaves)."""
    tq, tk, tv = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    scores = tq @ tk.transpose(-1, -2) / np.sqrt(q.shape[-1])
    if mask is not None:
        scores = scores.masked_fill(torch.tensor(mask), float(np.finfo(np.float32).min))
    w = torch.softmax(scores, -1)
    torch.manual_seed(seed)
    wd = F.dropout(w, rate, training=True)
    keep = (wd != 0).detach().numpy()
    return wd @ tv, keep, (tq, tk, tv)


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("rate", [0.1, 0.5])
def test_dropout_matches_torch_dropout_under_autograd(rate, masked):
    """The dropout branch (layers.py:537-544) against torch's own ``F.dropout`` on the softmax
    weights (which scales kept weights by 1 / (1 - rate), as flax's Dropout does), outputs and the
    three gradients under float64 autograd, with the keep mask torch drew."""
    q, k, v = _qkv(21, (2, 3, 10, 8))
    mask = None
    if masked:
        mask = np.zeros((10, 10), bool)
        mask[:, -2:] = True
        mask[4] = True
    out, keep, (tq, tk, tv) = _torch_dropout_attention(q, k, v, mask, rate, 5)
    assert 0 < keep.sum() < keep.size
    g = np.random.default_rng(3).standard_normal(q.shape)
    out.backward(torch.tensor(g))
    assert_close(AT.sdpa(q, k, v, mask, keep, rate), out.detach().numpy(), 1e-12, "out")
    for name, mine, want in zip("qkv", AT.sdpa_vjp(q, k, v, g, mask, keep, rate), (tq.grad, tk.grad, tv.grad)):
        assert_close(mine, want.numpy(), 1e-12, f"d{name}")


def test_dropout_closed_forms():
    """Every weight kept: the plain attention scaled by 1 / (1 - rate); rate 0 with any mask of ones:
    the plain attention; every weight dropped: zeros, and zero gradients."""
    q, k, v = _qkv(22, (1, 2, 7, 4))
    g = np.random.default_rng(4).standard_normal(q.shape)
    ones = np.ones((1, 2, 7, 7), bool)
    assert_close(AT.sdpa(q, k, v, None, ones, 0.25), AT.sdpa(q, k, v) / 0.75, 1e-12, "all kept")
    assert_close(AT.sdpa(q, k, v, None, ones, 0.0), AT.sdpa(q, k, v), 1e-12, "rate 0")
    assert not AT.sdpa(q, k, v, None, ~ones, 0.25).any()
    assert all(not t.any() for t in AT.sdpa_vjp(q, k, v, g, None, ~ones, 0.25))


@pytest.mark.parametrize("mistake", ["scale_by_rate", "drop_before_softmax", "vjp_without_keep"])
def test_dropout_planted_mistakes_are_caught(mistake, monkeypatch):
    if mistake == "scale_by_rate":
        monkeypatch.setattr(AT, "_dropped", lambda p, keep, rate: p if keep is None else np.where(keep, p / rate, 0.0))
    elif mistake == "drop_before_softmax":
        orig = AT._probs

        def bad_probs(q_, k_, mask):
            return orig(q_, k_, mask)

        def bad_dropped(p, keep, rate):  # renormalise the kept weights, as dropping scores would
            if keep is None:
                return p
            w = np.where(keep, p, 0.0)
            return w / w.sum(-1, keepdims=True)
        monkeypatch.setattr(AT, "_probs", bad_probs)
        monkeypatch.setattr(AT, "_dropped", bad_dropped)
    else:
        orig = AT._dropped
        calls = []

        def once(p, keep, rate):  # the VJP's second use (dP) without the mask
            calls.append(1)
            return orig(p, keep, rate) if len(calls) % 2 == 1 else p
        monkeypatch.setattr(AT, "_dropped", once)
    with pytest.raises(AssertionError):
        test_dropout_matches_torch_dropout_under_autograd(0.1, False)
