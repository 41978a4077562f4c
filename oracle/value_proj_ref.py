"""CPU oracle for MSDeformAttn's value projection with its epilogue — TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may use it, and only as the checker.

It restates, in NumPy (float64 from the given inputs):

* ``value_proj_rows``: ``Linear`` (src/rfdetr_jax/models/layers.py:258-280: ``x @ W^T + b`` with
  ``W [out, in]``), the padding mask ``where(mask[..., None], 0, value)`` (ops.py:377-379) and the
  head split ``[B, S, H*D] -> [B, S, H, D] -> [B, H, S, D] -> [B*H, S, D]`` (ops.py:405-407);
* ``value_proj_rows_vjp``: its transpose: ``dY`` is the cotangent read back through the head split
  with padded rows zeroed; ``dX = dY W``, ``dW = dY^T X``, ``db = sum dY``.

Pinning (tests/test_value_proj_oracle.py): torch float64 ``F.linear`` + ``masked_fill`` +
``permute`` under autograd (forward and all three gradients); closed forms (an identity weight copies
the input channels into the heads in order; a padded row is zero whatever the bias); planted
mistakes (heads and positions swapped in the split, the mask applied before the bias) fail them.
"""

from __future__ import annotations

import numpy as np

__all__ = ["value_proj_rows", "value_proj_rows_vjp"]


def value_proj_rows(x, weight, bias, n_heads, padding_mask=None):
    """``x [B, S, K]``, ``weight [N, K]``, ``bias [N]`` or None -> ``[B * H, S, N / H]`` float64."""
    x = np.asarray(x, np.float64)
    b, s, _ = x.shape
    y = x @ np.asarray(weight, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    if padding_mask is not None:
        y = np.where(np.asarray(padding_mask, bool)[..., None], 0.0, y)
    n = y.shape[-1]
    d = n // n_heads
    return y.reshape(b, s, n_heads, d).transpose(0, 2, 1, 3).reshape(b * n_heads, s, d)


def value_proj_rows_vjp(x, weight, n_heads, grad_value, padding_mask=None):
    """``(grad_x [B, S, K], grad_weight [N, K], grad_bias [N])`` float64."""
    x = np.asarray(x, np.float64)
    b, s, k = x.shape
    gv = np.asarray(grad_value, np.float64)
    d = gv.shape[-1]
    dy = gv.reshape(b, n_heads, s, d).transpose(0, 2, 1, 3).reshape(b, s, n_heads * d)
    if padding_mask is not None:
        dy = np.where(np.asarray(padding_mask, bool)[..., None], 0.0, dy)
    w = np.asarray(weight, np.float64)
    gx = dy @ w
    gw = dy.reshape(-1, n_heads * d).T @ x.reshape(-1, k)
    gb = dy.reshape(-1, n_heads * d).sum(0)
    return gx, gw, gb
