"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs on any host: the oracle against golden vectors and independent references,
the host-side argument handling, and the C ABI's exports and argument validation (no kernel runs).
``-m gpu`` runs the parity tests of the HIP kernels on an MI355X.
"""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "rf-detr-jax_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


import pytest  # noqa: E402


@pytest.fixture
def tune():
    """``tune({"MSDA_BWD_BANDS": 7})`` overrides launch-tuning knobs of the HIP library until the
    test ends (the library reads MSDA_* environment variables only once per process)."""
    from rfdetr_jax_amd import _native

    names = []

    def set_(knobs):
        for name, value in knobs.items():
            _native.check(_native.lib().msda_set_tuning(name.encode(), str(value).encode()))
            names.append(name)

    yield set_
    for name in names:
        _native.lib().msda_set_tuning(name.encode(), None)
