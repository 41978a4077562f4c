"""The forward's channel split on an MI355X: value levels too large for the LDS at head_dim channels,
staged at a half or a quarter of each head's channels per workgroup.

The library splits f32 value maps with at least 1024 queries by default; the tuning knob
MSDA_FWD_SPLIT forces the split (1) or the L2 gather of the large level (0). Each case runs the
forward twice, with the split and without it. Both compute every output channel with
the same operations in the same order, so the outputs must be bit-identical; the split output is
also checked against the float64 oracle. The cases cover one and two chunks of 16 bytes per staged
cell, a split by two and by four, f32 and bf16 value maps, a level that fills the LDS, query counts
on both sides of the planner's head grouping, the bf16 samplers' rounding points and the fused
prologue.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import msda_ref as R
from oracle import prologue_ref as PR
from rfdetr_jax_amd import _native
from rfdetr_jax_amd import ops as hip
from rfdetr_jax_amd.workloads import make_fused_inputs, make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu

# name: (value dtype, head_dim, level shapes, points, queries, batch, heads)
CASES = {
    "bf16_d16_two_levels_half": ("bf16", 16, ((80, 80), (20, 20)), 4, 300, 2, 4),
    "bf16_d32_quarter": ("bf16", 32, ((80, 80),), 2, 300, 1, 4),
    "f32_d16_half_two_chunks": ("f32", 16, ((64, 64), (8, 8)), 4, 300, 2, 2),
    "f32_d32_quarter_two_chunks": ("f32", 32, ((64, 64),), 2, 200, 1, 4),
    "f32_d8_half_fills_lds": ("f32", 8, ((100, 100),), 2, 300, 1, 2),
    "bf16_d16_many_queries": ("bf16", 16, ((80, 80),), 2, 3900, 1, 8),
    "f32_d16_split_by_default": ("f32", 16, ((64, 64), (32, 32)), 4, 1200, 1, 4),
}


def _note(msg):
    sys.stderr.write(f"[gpu] {msg}\n")
    sys.stderr.flush()


def _both(fn):
    """fn() with the channel split, then without it."""
    with _native.tuning({"MSDA_FWD_SPLIT": 1}):
        split = fn()
    with _native.tuning({"MSDA_FWD_SPLIT": 0}):
        plain = fn()
    torch.cuda.synchronize()
    return split, plain


@pytest.mark.parametrize("case", list(CASES))
def test_split_forward_matches_the_gathered_one_and_the_oracle(case):
    dtype, d, shapes, p, q, b, h = CASES[case]
    _note(f"channel split {case}")
    value, loc, attn, _ = make_inputs(40 + len(case), b, h, d, q, shapes, p)
    dev = torch.device("cuda:0")
    if dtype == "bf16":
        value = R.bf16_round(value)
        v = torch.from_numpy(value).to(dev).to(torch.bfloat16)
    else:
        v = torch.from_numpy(value).to(dev)
    lc, a = torch.from_numpy(loc).to(dev), torch.from_numpy(attn).to(dev)
    split, plain = _both(lambda: hip.ms_deform_attn_forward(v, shapes, lc, a))
    assert torch.equal(split, plain)
    assert_close(split.cpu().numpy(), R.ms_deform_attn_core_rows(value, shapes, loc, attn), 1e-5, "out")


@pytest.mark.parametrize("sampler", ["gather", "gather-f32", "matmul"])
def test_split_forward_keeps_the_samplers_rounding_points(sampler):
    shapes = ((80, 80), (20, 20))
    _note(f"channel split sampler={sampler}")
    value, loc, attn, _ = make_inputs(9, 2, 4, 16, 300, shapes, 4)
    value = R.bf16_round(value)
    dev = torch.device("cuda:0")
    v = torch.from_numpy(value).to(dev).to(torch.bfloat16)
    lc, a = torch.from_numpy(loc).to(dev), torch.from_numpy(attn).to(dev)
    split, plain = _both(lambda: hip.ms_deform_attn_forward(v, shapes, lc, a, sampler=sampler))
    assert torch.equal(split, plain)
    want = R.ms_deform_attn_core_rows_sampler(value, shapes, loc, attn, sampler, True)
    assert_close(split.cpu().numpy(), want, 2e-6, f"{sampler} forward")


@pytest.mark.parametrize("ref_dim", [2, 4])
def test_split_fused_forward(ref_dim):
    shapes = ((80, 80), (20, 20))
    _note(f"channel split fused ref_dim={ref_dim}")
    value, ref, off, logits, _ = make_fused_inputs(12, 2, 4, 16, 300, shapes, 4, ref_dim)
    dev = torch.device("cuda:0")
    v = torch.from_numpy(R.bf16_round(value)).to(dev).to(torch.bfloat16)
    r, o, lg = (torch.from_numpy(x).to(dev) for x in (ref, off, logits))
    split, plain = _both(lambda: hip.ms_deform_attn_fused_forward(v, shapes, r, o, lg))
    assert torch.equal(split, plain)
    loc, attn = PR.prologue(ref, off, logits, shapes, 4)
    want = R.ms_deform_attn_core_rows(R.bf16_round(value), shapes, loc, attn)
    assert_close(split.cpu().numpy(), want, 1e-5, "fused out")


def test_split_forward_in_a_batch_with_a_narrow_output_dtype():
    """bf16 output rows written by the parts of a split head (16-byte runs of 8 channels)."""
    shapes = ((80, 80),)
    value, loc, attn, _ = make_inputs(13, 2, 2, 16, 300, shapes, 2)
    value = R.bf16_round(value)
    dev = torch.device("cuda:0")
    v = torch.from_numpy(value).to(dev).to(torch.bfloat16)
    lc, a = torch.from_numpy(loc).to(dev), torch.from_numpy(attn).to(dev)
    split, plain = _both(lambda: hip.ms_deform_attn_forward(v, shapes, lc, a, out_dtype=torch.bfloat16))
    assert split.dtype == torch.bfloat16
    assert torch.equal(split, plain)
    want = R.ms_deform_attn_core_rows(value, shapes, loc, attn)
    assert_close(split.float().cpu().numpy(), want, 1e-2, "bf16 out")
    assert bool(np.isfinite(split.float().cpu().numpy()).all())
