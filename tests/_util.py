"""Shared helpers for the tests (fixture loading, tolerance checks)."""

from __future__ import annotations

import glob
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden_names():
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


def load_golden(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        data = {k: z[k] for k in z.files}
    data["meta"] = json.loads(str(data["meta"]))
    data["shapes"] = tuple((int(h), int(w)) for h, w in data["shapes"])
    return data


def assert_close(got, want, tol, what=""):
    """``max|got - want| <= tol * max(1, max|want|)`` — the reference's gradient criterion
    (tests/test_ops.py:245-248), used here for every output."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if want.size == 0:
        return
    err = float(np.max(np.abs(got - want)))
    bound = tol * max(1.0, float(np.max(np.abs(want))))
    assert err <= bound, f"{what}: max|diff| = {err:.3e} > {bound:.3e}"
