"""Parity of the decoder self-attention kernels (msda_attention_fwd / _bwd through the C ABI, via
the torch mirror rfdetr_jax_amd.attention) on an MI355X.

Expected values: oracle/attention_ref.py (float64); for the module, torch's
``nn.MultiheadAttention`` in float64 on the CPU, run per (image, group). Tolerances
(``max|got - want| <= tol * max(1, max|want|)``): f32 forward 1e-5, gradients 1e-4; bf16 2e-2.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import attention_ref as AT
from oracle.msda_ref import bf16_round
from rfdetr_jax_amd.attention import (
    MultiheadAttention,
    decoder_self_attention,
    grouped_attention,
    scaled_dot_product_attention,
)
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
    "decoder": (6, 8, 300, 32),   # 300 queries per group, 8 heads x 32 (config-2 slices, fewer of them)
    "small": (2, 3, 9, 32),
    "ragged": (2, 2, 37, 64),     # head_dim 64, rows not a multiple of 32
    "one": (1, 1, 1, 32),
    "long": (1, 2, 480, 32),      # 8 chunks of keys
    "long64": (1, 1, 1000, 64),   # head_dim 64, 16 chunks
}


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_sdpa_against_oracle(shape, masked, bf16):
    b, h, length, d = SHAPES[shape]
    _note(f"sdpa {shape} masked={masked} bf16={bf16}")
    rng = np.random.default_rng(41)
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    mask = None
    if masked:
        mask = rng.uniform(0, 1, (length, length)) < 0.2
        mask[:, -3:] = True  # tests/test_attention.py:37-40
        mask[length // 2] = True  # a fully blocked row: uniform weights
    if bf16:
        q, k, v, g = (bf16_round(t) for t in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else None
    tq, tk, tv = (_t(x, dt).requires_grad_(True) for x in (q, k, v))
    out = scaled_dot_product_attention(tq, tk, tv, None if mask is None else _t(mask))
    out.backward(_t(g, dt))
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), AT.sdpa(q, k, v, mask), tf, "out")
    for name, t, want in zip("qkv", (tq, tk, tv), AT.sdpa_vjp(q, k, v, g, mask)):
        assert_close(_np(t.grad), want, tg, f"grad_{name}")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("order", ["rising", "falling"])
def test_sdpa_reference_score_moves(order, bf16):
    """The forward's running reference score moves only when a key chunk's maximum exceeds it by
    more than 8 (log2 units). Keys scaled up chunk by chunk (factors 1, 4, 7, 10, 13) move it at
    every chunk, with the partial sums rescaled each time; scaled down, it never moves after the
    first chunk and later weights are far below 1."""
    b, h, length, d = 2, 4, 300, 32
    _note(f"sdpa reference score {order} bf16={bf16}")
    rng = np.random.default_rng(43)
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    factor = 1.0 + 3.0 * (np.arange(length) // 64)
    k = k * (factor if order == "rising" else factor[::-1])[:, None].astype(np.float32)
    if bf16:
        q, k, v, g = (bf16_round(t) for t in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else None
    tq, tk, tv = (_t(x, dt).requires_grad_(True) for x in (q, k, v))
    out = scaled_dot_product_attention(tq, tk, tv)
    out.backward(_t(g, dt))
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), AT.sdpa(q, k, v, None), tf, "out")
    for name, t, want in zip("qkv", (tq, tk, tv), AT.sdpa_vjp(q, k, v, g, None)):
        assert_close(_np(t.grad), want, tg, f"grad_{name}")


def test_reference_known_answers():
    """tests/test_attention.py:104-119 (at head_dim 32): equal scores give the mean of V, and the
    padding of the key blocks takes no weight."""
    q = torch.ones((2, 3, 145, 32), device=_dev())
    k = -torch.ones((2, 3, 145, 32), device=_dev())
    v = _t(np.random.default_rng(0).standard_normal((2, 3, 145, 32)).astype(np.float32))
    out = _np(scaled_dot_product_attention(q, k, v))
    want = _np(v).astype(np.float64).mean(axis=2, keepdims=True)
    assert_close(out, np.broadcast_to(want, out.shape), 1e-5, "mean")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_grouped_rows_layout_against_split_groups(bf16):
    """[B, G * P, C] rows with q and k read in place from a fused [B, Q, 2C] projection (row stride
    2C): the same as splitting the groups onto the batch, attending per head and merging back."""
    batch, groups, per, heads, d = 2, 13, 30, 8, 32
    c = heads * d
    _note(f"grouped rows bf16={bf16}")
    rng = np.random.default_rng(42)
    qk = rng.standard_normal((batch, groups * per, 2 * c)).astype(np.float32)
    v = rng.standard_normal((batch, groups * per, c)).astype(np.float32)
    g = rng.standard_normal((batch, groups * per, c)).astype(np.float32)
    if bf16:
        qk, v, g = (bf16_round(x) for x in (qk, v, g))
    dt = torch.bfloat16 if bf16 else None
    tqk = _t(qk, dt).requires_grad_(True)
    tv = _t(v, dt).requires_grad_(True)
    out = grouped_attention(tqk[..., :c], tqk[..., c:], tv, heads, groups)
    out.backward(_t(g, dt))
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)

    def heads_of(x):  # [G B, P, C] -> [G B, H, P, D]
        return x.reshape(x.shape[0], per, heads, d).transpose(0, 2, 1, 3)

    qs, ks, vs = (heads_of(AT.split_groups(x, per)) for x in (qk[..., :c], qk[..., c:], v))
    gs = heads_of(AT.split_groups(g, per))
    want = AT.merge_groups(AT.sdpa(qs, ks, vs).transpose(0, 2, 1, 3).reshape(groups * batch, per, c), batch)
    assert_close(_np(out), want, tf, "out")
    dq, dk, dv = (AT.merge_groups(x.transpose(0, 2, 1, 3).reshape(groups * batch, per, c), batch) for x in AT.sdpa_vjp(qs, ks, vs, gs))
    gqk = _np(tqk.grad)
    assert_close(gqk[..., :c], dq, tg, "grad_q")
    assert_close(gqk[..., c:], dk, tg, "grad_k")
    assert_close(_np(tv.grad), dv, tg, "grad_v")


def _torch_reference(m, tgt, pos, groups, heads, grad):
    """The decoder self-attention written with torch's float64 nn.MultiheadAttention on the CPU, one
    (image, group) block at a time, with the parameter gradients."""
    c = tgt.shape[-1]
    ref = torch.nn.MultiheadAttention(c, heads, batch_first=True, dtype=torch.float64)
    with torch.no_grad():
        ref.in_proj_weight.copy_(m.in_proj_weight.detach().double().cpu())
        ref.in_proj_bias.copy_(m.in_proj_bias.detach().double().cpu())
        ref.out_proj.weight.copy_(m.out_proj.weight.detach().double().cpu())
        ref.out_proj.bias.copy_(m.out_proj.bias.detach().double().cpu())
    t = torch.tensor(tgt, dtype=torch.float64, requires_grad=True)
    p = torch.tensor(pos, dtype=torch.float64)
    batch, total, _ = tgt.shape
    per = total // groups
    query = t + p
    outs = []
    for b in range(batch):
        row = []
        for g in range(groups):
            sl = slice(g * per, (g + 1) * per)
            o, _ = ref(query[b:b + 1, sl], query[b:b + 1, sl], t[b:b + 1, sl], need_weights=False)
            row.append(o)
        outs.append(torch.cat(row, 1))
    out = torch.cat(outs, 0)
    out.backward(torch.tensor(grad, dtype=torch.float64))
    grads = {"in_proj_weight": ref.in_proj_weight.grad, "in_proj_bias": ref.in_proj_bias.grad,
             "out_proj.weight": ref.out_proj.weight.grad, "out_proj.bias": ref.out_proj.bias.grad}
    return out.detach().numpy(), t.grad.numpy(), {k: v.numpy() for k, v in grads.items()}


@pytest.mark.parametrize("groups", [1, 3])
def test_decoder_self_attention_module(groups):
    """The whole block (fused q/k projection, attention per group, out_proj) and every gradient."""
    torch.manual_seed(0)
    heads, c, batch, per = 8, 256, 2, 40
    m = MultiheadAttention(c, heads).to(_dev())
    with torch.no_grad():
        m.in_proj_bias.normal_(0, 0.1)
        m.out_proj.bias.normal_(0, 0.1)
    rng = np.random.default_rng(43)
    tgt = rng.standard_normal((batch, groups * per, c)).astype(np.float32)
    pos = rng.standard_normal((batch, groups * per, c)).astype(np.float32)
    grad = rng.standard_normal((batch, groups * per, c)).astype(np.float32)
    tt = _t(tgt).requires_grad_(True)
    out = decoder_self_attention(tt, _t(pos), m, groups)
    out.backward(_t(grad))
    want, want_dt, want_grads = _torch_reference(m, tgt, pos, groups, heads, grad)
    assert_close(_np(out), want, 1e-5, "out")
    assert_close(_np(tt.grad), want_dt, 1e-4, "grad tgt")
    for name, p in m.named_parameters():
        assert_close(_np(p.grad), want_grads[name], 1e-4, f"grad {name}")


def test_single_gradient_requests():
    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    rng = np.random.default_rng(44)
    q, k, v, g = (rng.standard_normal((2, 2, 50, 32)).astype(np.float32) for _ in range(4))
    lay = _Layout(2, 1, 2, 50, 32)
    tq, tk, tv = _t(q), _t(k), _t(v)
    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    want = AT.sdpa_vjp(q, k, v, g)
    for i in range(3):
        needs = tuple(j == i for j in range(3))
        got = attention_backward(tq, tk, tv, out, stats, _t(g), lay, lay.strides_bhld, None, needs)
        for j in range(3):
            if j == i:
                assert_close(_np(got[j]), want[j], 1e-4, f"gradient {j}")
            else:
                assert got[j] is None


FUSED_LENGTHS = [1, 17, 32, 33, 64, 65, 129, 200, 256, 257, 300, 319, 320, 321]


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("length", FUSED_LENGTHS)
def test_fused_backward_against_two_kernel_path(length, bf16, tune):
    """Head_dim 32 without a mask, up to 320 rows: one fused backward kernel (one workgroup per
    (slice, head): a wave per key block, two waves that form dQ from the dS tiles) against the
    oracle, and against the two-kernel path (MSDA_ATTN_FUSED=0) on the same forward; both write
    rowsum(dO * O) into entry 2 of the statistics. 321 rows take the two kernels either way."""
    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    b, h, d = 2, 3, 32
    _note(f"fused backward L={length} bf16={bf16}")
    rng = np.random.default_rng(45 + length)
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else torch.float32
    tol, cross = (2e-2, 1e-2) if bf16 else (1e-4, 1e-4)
    lay = _Layout(b, 1, h, length, d)
    tq, tk, tv, tg = (_t(x, dt) for x in (q, k, v, g))
    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    fused = attention_backward(tq, tk, tv, out, stats, tg, lay, lay.strides_bhld)
    torch.cuda.synchronize()
    dsum_fused = _np(stats).reshape(b * h * length, 4)[:, 2].copy()
    tune({"MSDA_ATTN_FUSED": 0})
    split = attention_backward(tq, tk, tv, out, stats, tg, lay, lay.strides_bhld)
    torch.cuda.synchronize()
    dsum_split = _np(stats).reshape(b * h * length, 4)[:, 2]
    want_dsum = (g.astype(np.float64) * _np(out).astype(np.float64)).sum(-1).reshape(-1)
    assert_close(dsum_fused, want_dsum, 1e-5, "rowsum(dO * O), fused")
    assert_close(dsum_split, want_dsum, 1e-5, "rowsum(dO * O), two kernels")
    want = AT.sdpa_vjp(q, k, v, g)
    for name, a, c, w in zip("qkv", fused, split, want):
        assert_close(_np(a), w, tol, f"grad_{name} fused")
        assert_close(_np(c), w, tol, f"grad_{name} two kernels")
        assert_close(_np(a), _np(c).astype(np.float64), cross, f"grad_{name} fused against two kernels")


D32_LENGTHS = [1, 17, 63, 64, 65, 128, 129, 300, 320, 321, 480, 512, 513]


@pytest.mark.parametrize("length", D32_LENGTHS)
def test_bf16_forward_d32_against_chunked(length, tune):
    """bf16, head_dim 32, no mask, 16-byte aligned key and value rows, up to 512 rows: the forward
    that stages the whole key and value slice in LDS (scores leave the MFMA scaled and shifted,
    row sums add the rounded weights) against the oracle and the chunked kernel
    (MSDA_ATTN_FWD_D32=0). Its statistics give log2 sum_k 2^x (x = q.k log2(e) / sqrt(D)) as
    m + log2 l, and drive the backward. 513 rows take the chunked kernel either way."""
    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    b, h, d = 2, 3, 32
    _note(f"bf16 forward d32 L={length}")
    rng = np.random.default_rng(47 + length)
    q, k, v, g = (bf16_round(rng.standard_normal((b, h, length, d)).astype(np.float32)) for _ in range(4))
    lay = _Layout(b, 1, h, length, d)
    tq, tk, tv, tg = (_t(x, torch.bfloat16) for x in (q, k, v, g))
    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    grads = attention_backward(tq, tk, tv, out, stats, tg, lay, lay.strides_bhld)
    torch.cuda.synchronize()
    st = _np(stats).reshape(b, h, length, 4)
    tune({"MSDA_ATTN_FWD_D32": 0})
    out2, _ = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    torch.cuda.synchronize()
    assert_close(_np(out), AT.sdpa(q, k, v, None), 2e-2, "out")
    assert_close(_np(out), _np(out2).astype(np.float64), 1e-2, "out against the chunked kernel")
    x = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)) * (np.log2(np.e) / np.sqrt(d))
    xm = x.max(-1)
    lse2 = xm + np.log2(np.exp2(x - xm[..., None]).sum(-1))
    err = np.abs(st[..., 0] + st[..., 1] - lse2).max()
    assert err <= 1e-2, f"m + log2 l against log2 sum 2^x: max error {err}"
    for name, a, w in zip("qkv", grads, AT.sdpa_vjp(q, k, v, g)):
        assert_close(_np(a), w, 2e-2, f"grad_{name}")


@pytest.mark.parametrize("case", ["far_below", "unaligned_rows"])
def test_bf16_forward_d32_edge_cases(case, tune):
    """far_below: every score about -65 (log2 units), below the reference score's low limit, so it
    moves at the first chunk; equal scores give the mean of V. unaligned_rows: key and value rows
    with a stride of 36 elements (not 16-byte aligned) take the chunked kernel."""
    from rfdetr_jax_amd.attention import _Layout, attention_forward

    _note(f"bf16 forward d32 {case}")
    b, h, length, d = 2, 2, 200, 32
    rng = np.random.default_rng(48)
    v = bf16_round(rng.standard_normal((b, h, length, d)).astype(np.float32))
    if case == "far_below":
        q = np.full((b, h, length, d), 8.0, np.float32)
        k = -np.ones((b, h, length, d), np.float32)
        lay = _Layout(b, 1, h, length, d)
        out, _ = attention_forward(_t(q, torch.bfloat16), _t(k, torch.bfloat16), _t(v, torch.bfloat16), lay, lay.strides_bhld)
        want = np.broadcast_to(v.astype(np.float64).mean(axis=2, keepdims=True), v.shape)
        assert_close(_np(out), want, 2e-2, "mean of V")
        return
    q, k = (bf16_round(rng.standard_normal((b, h, length, d)).astype(np.float32)) for _ in range(2))
    pad = np.zeros((b, h, length, 36), np.float32)
    tq = _t(q, torch.bfloat16)
    tk = _t(np.concatenate([k, pad[..., :4]], -1), torch.bfloat16)[..., :d]
    tv = _t(np.concatenate([v, pad[..., :4]], -1), torch.bfloat16)[..., :d]
    lay = _Layout(b, 1, h, length, d)
    out, _ = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    assert_close(_np(out), AT.sdpa(q, k, v, None), 2e-2, "out")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("needs", [(True, True, False), (True, False, True), (True, False, False), (False, True, True)],
                         ids=["qk", "qv", "q", "kv"])
def test_gradient_subsets_head_dim_32(needs, bf16):
    """Head_dim 32: grad_q with one of grad_k / grad_v (the fused kernel, skipping the missing
    store), grad_q alone and grad_k with grad_v (the two-kernel path's halves)."""
    from rfdetr_jax_amd.attention import _Layout, attention_backward, attention_forward

    _note(f"gradient subset {needs} bf16={bf16}")
    rng = np.random.default_rng(46)
    q, k, v, g = (rng.standard_normal((2, 2, 150, 32)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else torch.float32
    lay = _Layout(2, 1, 2, 150, 32)
    tq, tk, tv = (_t(x, dt) for x in (q, k, v))
    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    got = attention_backward(tq, tk, tv, out, stats, _t(g, dt), lay, lay.strides_bhld, None, needs)
    torch.cuda.synchronize()
    want = AT.sdpa_vjp(q, k, v, g)
    for j in range(3):
        if needs[j]:
            assert_close(_np(got[j]), want[j], 2e-2 if bf16 else 1e-4, f"gradient {j}")
        else:
            assert got[j] is None


@pytest.mark.parametrize("path", ["bf16", "bf16-two-kernels", "f32"])
def test_unaligned_output_rows(path, tune):
    """Every kernel stores its results as 16-byte row pieces through an LDS transpose when the
    output rows allow it, element by element otherwise. Here the forward output and the gradients
    start 8 bytes (bf16) or 4 bytes (f32) into a buffer, with a row stride of 36 elements; the
    elements between the rows stay untouched."""
    import ctypes

    from rfdetr_jax_amd import _native
    from rfdetr_jax_amd.attention import _DTYPES, _Layout, _ptr, _stream, attention_forward

    bf16 = path != "f32"
    if path == "bf16-two-kernels":
        tune({"MSDA_ATTN_FUSED": 0})
    b, h, length, d, rs = 2, 3, 300, 32, 36
    off = 4 if bf16 else 1
    dt = torch.bfloat16 if bf16 else torch.float32
    _note(f"unaligned output rows {path}")
    rng = np.random.default_rng(47)
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    lay = _Layout(b, 1, h, length, d)
    tq, tk, tv, tg = (_t(x, dt) for x in (q, k, v, g))
    n = b * h * length * rs
    row_strides = [h * length * rs, 0, length * rs, rs]

    def views(count):
        bufs = [torch.zeros(n + off, dtype=dt, device=_dev()) for _ in range(count)]
        return bufs, [x[off:].view(b, h, length, rs)[..., :d] for x in bufs]

    def untouched(bufs):
        for x in bufs:
            assert not _np(x[off:].view(b, h, length, rs)[..., d:]).any() and not _np(x[:off]).any()

    tf, tg_ = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    obufs, (out_u,) = views(1)
    stats_u = torch.empty(b * h * length * 4, dtype=torch.float32, device=_dev())
    s = lay.strides_bhld(tq) + lay.strides_bhld(tk) + lay.strides_bhld(tv) + row_strides
    rc = _native.lib().msda_attention_fwd(_ptr(tq), _ptr(tk), _ptr(tv), _DTYPES[dt], _ptr(out_u), _ptr(stats_u), b, 1, h, length, d,
                                          (ctypes.c_int64 * 16)(*s), None, _stream(_dev()))
    _native.check(rc)
    torch.cuda.synchronize()
    assert_close(_np(out_u), AT.sdpa(q, k, v, None), tf, "out")
    untouched(obufs)

    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    gbufs, grads = views(3)
    s = []
    for t in (tq, tk, tv, out, tg):
        s += lay.strides_bhld(t)
    for _ in grads:
        s += row_strides
    rc = _native.lib().msda_attention_bwd(_ptr(tq), _ptr(tk), _ptr(tv), _ptr(out), _ptr(stats), _ptr(tg), _DTYPES[dt],
                                          _ptr(grads[0]), _ptr(grads[1]), _ptr(grads[2]), b, 1, h, length, d,
                                          (ctypes.c_int64 * 32)(*s), None, _stream(_dev()))
    _native.check(rc)
    torch.cuda.synchronize()
    for name, got, want in zip("qkv", grads, AT.sdpa_vjp(q, k, v, g)):
        assert_close(_np(got), want, tg_, f"grad_{name}")
    untouched(gbufs)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("seed", range(6))
def test_fused_backward_random_shapes(seed, bf16):
    """Seeded random shapes through the fused backward (head_dim 32, no mask): 1-3 images, 1-4
    heads, 1-320 rows, rows padded to a random stride (a multiple of 4 elements, as the interface
    requires), against the float64 oracle."""
    import ctypes

    from rfdetr_jax_amd import _native
    from rfdetr_jax_amd.attention import _DTYPES, _Layout, _ptr, _stream, attention_forward

    rng = np.random.default_rng(1000 + seed)
    b, h, length, d = int(rng.integers(1, 4)), int(rng.integers(1, 5)), int(rng.integers(1, 321)), 32
    rs = d + 4 * int(rng.integers(0, 4))
    _note(f"fused random shape seed={seed} bf16={bf16}: b={b} h={h} L={length} row stride {rs}")
    dt = torch.bfloat16 if bf16 else torch.float32
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))

    def padded(x):
        buf = torch.zeros((b, h, length, rs), dtype=dt, device=_dev())
        if x is not None:
            buf[..., :d] = _t(x, dt)
        return buf[..., :d]

    tq, tk, tv, tg = (padded(x) for x in (q, k, v, g))
    lay = _Layout(b, 1, h, length, d)
    out, stats = attention_forward(tq, tk, tv, lay, lay.strides_bhld)
    grads = [padded(None) for _ in range(3)]
    s = []
    for t in (tq, tk, tv, out, tg, *grads):
        s += lay.strides_bhld(t)
    rc = _native.lib().msda_attention_bwd(_ptr(tq), _ptr(tk), _ptr(tv), _ptr(out), _ptr(stats), _ptr(tg), _DTYPES[dt],
                                          _ptr(grads[0]), _ptr(grads[1]), _ptr(grads[2]), b, 1, h, length, d,
                                          (ctypes.c_int64 * 32)(*s), None, _stream(_dev()))
    _native.check(rc)
    torch.cuda.synchronize()
    for name, got, want in zip("qkv", grads, AT.sdpa_vjp(q, k, v, g)):
        assert_close(_np(got), want, 2e-2 if bf16 else 1e-4, f"grad_{name}")


# --------------------------------------------------------------------------------------------
# attention dropout (layers.py:537-544): the keep decisions come from dropout_keep_mask, the same
# hash the kernels evaluate; the expected values are the float64 oracle with that mask.

DROP_SHAPES = {
    "decoder": (3, 8, 300, 32),
    "ragged64": (2, 2, 77, 64),
    "one": (1, 1, 1, 32),
}


def _keep(batch, heads, length, rate, seed, groups=1):
    from rfdetr_jax_amd.attention import dropout_keep_mask

    return dropout_keep_mask(batch, heads, length, rate, seed, groups=groups, device=_dev())


def test_dropout_keep_mask_statistics():
    """Keep rate 1 - rate (overall, for even and odd keys, which share one hash, and across
    neighbouring queries, within six standard deviations); the same (rate, seed) gives the same
    mask, another seed or another slice an independent one (disagreement 2 r (1 - r))."""
    b, h, length = 4, 8, 300
    for rate in (0.1, 0.5, 0.9):
        keep = _keep(b, h, length, rate, 1234).float()
        n = keep.numel()
        sd = (rate * (1 - rate) / n) ** 0.5
        _note(f"dropout rate {rate}: kept {keep.mean().item():.5f}")
        assert abs(keep.mean().item() - (1 - rate)) < 6 * sd
        for part in (keep[..., 0::2], keep[..., 1::2]):
            assert abs(part.mean().item() - (1 - rate)) < 6 * sd * 2 ** 0.5
        both = (keep[..., 0:298:2] * keep[..., 1:299:2]).mean().item()  # the two halves of one hash
        rows = (keep[:, :, 0::2, :] * keep[:, :, 1::2, :]).mean().item()
        sd2 = ((1 - rate) ** 2 * (1 - (1 - rate) ** 2) / (n / 2)) ** 0.5
        assert abs(both - (1 - rate) ** 2) < 6 * sd2 and abs(rows - (1 - rate) ** 2) < 6 * sd2
    k1 = _keep(b, h, length, 0.1, 1234)
    assert torch.equal(k1, _keep(b, h, length, 0.1, 1234))
    other = (k1 != _keep(b, h, length, 0.1, 1235)).float().mean().item()
    slices = (k1[0, 0] != k1[0, 1]).float().mean().item()
    assert abs(other - 0.18) < 0.005 and abs(slices - 0.18) < 0.01
    assert bool((_keep(1, 2, 40, 0.0, 5) == 1).all())


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("shape", sorted(DROP_SHAPES))
def test_dropout_against_oracle(shape, masked, bf16):
    """Output and gradients with dropout (rate 0.1) against the float64 oracle given the kernels'
    keep mask, with and without a key mask (a fully blocked row included)."""
    b, h, length, d = DROP_SHAPES[shape]
    rate, seed = 0.1, 1000 + length
    _note(f"dropout {shape} masked={masked} bf16={bf16}")
    rng = np.random.default_rng(43)
    q, k, v, g = (rng.standard_normal((b, h, length, d)).astype(np.float32) for _ in range(4))
    mask = None
    if masked:
        mask = rng.uniform(0, 1, (length, length)) < 0.2
        mask[:, -3:] = True
        mask[length // 2] = True
    if bf16:
        q, k, v, g = (bf16_round(t) for t in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else None
    tq, tk, tv = (_t(x, dt).requires_grad_(True) for x in (q, k, v))
    out = scaled_dot_product_attention(tq, tk, tv, None if mask is None else _t(mask), dropout=rate, seed=seed)
    out.backward(_t(g, dt))
    keep = _np(_keep(b, h, length, rate, seed)).astype(bool)
    torch.cuda.synchronize()
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)
    assert_close(_np(out), AT.sdpa(q, k, v, mask, keep, rate), tf, "out")
    for name, t, want in zip("qkv", (tq, tk, tv), AT.sdpa_vjp(q, k, v, g, mask, keep, rate)):
        assert_close(_np(t.grad), want, tg, f"grad_{name}")


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_grouped_dropout_rows_layout(bf16):
    """Dropout on [B, G * P, C] rows with G groups: slice z = g * B + b of the keep mask belongs to
    group g of image b (the order of _split_groups)."""
    batch, groups, per, heads, d = 2, 3, 40, 4, 32
    c = heads * d
    rate, seed = 0.2, 9
    rng = np.random.default_rng(44)
    q, k, v, g = (rng.standard_normal((batch, groups * per, c)).astype(np.float32) for _ in range(4))
    if bf16:
        q, k, v, g = (bf16_round(x) for x in (q, k, v, g))
    dt = torch.bfloat16 if bf16 else None
    tq, tk, tv = (_t(x, dt).requires_grad_(True) for x in (q, k, v))
    out = grouped_attention(tq, tk, tv, heads, groups, dropout=rate, seed=seed)
    out.backward(_t(g, dt))
    keep = _np(_keep(batch, heads, per, rate, seed, groups=groups)).astype(bool)  # [G B, H, P, P]
    tf, tg = (2e-2, 2e-2) if bf16 else (1e-5, 1e-4)

    def heads_of(x):  # [G B, P, C] -> [G B, H, P, D]
        return x.reshape(x.shape[0], per, heads, d).transpose(0, 2, 1, 3)

    def back(x):  # [G B, H, P, D] -> [B, G P, C]
        return AT.merge_groups(x.transpose(0, 2, 1, 3).reshape(groups * batch, per, c), batch)

    qs, ks, vs, gs = (heads_of(AT.split_groups(x, per)) for x in (q, k, v, g))
    assert_close(_np(out), back(AT.sdpa(qs, ks, vs, None, keep, rate)), tf, "out")
    for name, t, want in zip("qkv", (tq, tk, tv), AT.sdpa_vjp(qs, ks, vs, gs, None, keep, rate)):
        assert_close(_np(t.grad), back(want), tg, f"grad_{name}")


def test_dropout_module_training_and_eval():
    """MultiheadAttention(dropout=0.1): in training a call draws its seed from torch's generator
    (repeatable under torch.manual_seed, different otherwise) and its gradients are finite; in
    eval the module is the plain attention; rate 0 is the plain path bit for bit; rate 1 gives
    zeros (flax's Dropout at rate 1)."""
    torch.manual_seed(0)
    m = MultiheadAttention(64, 2, dropout=0.1).to(_dev())
    x = torch.randn(2, 50, 64, device=_dev(), requires_grad=True)
    m.train()
    torch.manual_seed(5)
    y1 = m(x, x, x)
    torch.manual_seed(5)
    y2 = m(x, x, x)
    torch.manual_seed(6)
    y3 = m(x, x, x)
    assert torch.equal(y1, y2) and not torch.equal(y1, y3)
    y1.square().sum().backward()
    assert torch.isfinite(x.grad).all() and torch.isfinite(m.in_proj_weight.grad).all()
    m.eval()
    plain = MultiheadAttention(64, 2).to(_dev())
    plain.load_state_dict(m.state_dict())
    with torch.no_grad():
        assert torch.equal(m(x, x, x), plain(x, x, x))
    q, k, v = (torch.randn(1, 2, 33, 32, device=_dev()) for _ in range(3))
    assert torch.equal(scaled_dot_product_attention(q, k, v, dropout=0.0, seed=3), scaled_dot_product_attention(q, k, v))
    assert not scaled_dot_product_attention(q, k, v, dropout=1.0).any()
