"""Build the gfx950 HIP library ``libmsda_gfx950.so`` in-tree with hipcc.

``python -m rfdetr_jax_amd.build`` (with ``rf-detr-jax_amd/`` on ``sys.path``) or
``__graft_entry__.build()`` runs it. The library is placed next to this file, where
``rfdetr_jax_amd._native`` loads it from.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)  # rf-detr-jax_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_NAME = "libmsda_gfx950.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The C ABI, and the kernel instantiations split by value dtype and direction so they compile in
# parallel.
SOURCES = [os.path.join(CSRC, f) for f in ("msda_abi.hip", "msda_fwd_f32.hip", "msda_fwd_bf16.hip", "msda_bwd_f32.hip",
                                           "msda_bwd_bf16.hip", "grid_sample_abi.hip", "value_proj_abi.hip",
                                           "attention_abi.hip", "probe_abi.hip")]
HEADERS = [os.path.join(CSRC, f) for f in ("msda_kernels.h", "msda_band_kernels.h", "msda_gather_kernels.h", "msda_fused_bwd_kernels.h", "msda_launch.h", "grid_sample_kernels.h",
                                           "value_proj_kernels.h", "attention_kernels.h")] + [
    os.path.join(INCLUDE, "msda.h"), os.path.join(INCLUDE, "msda_probe.h")]
BUILD_DIR = os.path.join(ROOT, "_build")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Keep the compiler from forming packed-f32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}: {' '.join(cmd[-3:])}")
    if verbose and proc.stderr.strip():
        sys.stderr.write(proc.stderr)


def build(verbose: bool = False, extra_flags: list[str] | None = None, out: str | None = None) -> str:
    """Compile the library; returns its path. Always recompiles (it is the build check)."""
    out = out or LIB_PATH
    tmp = out + ".tmp"
    objdir = os.path.join(BUILD_DIR, os.path.basename(out) + ".objs")
    os.makedirs(objdir, exist_ok=True)
    flags = [*HIPCC_FLAGS, *(extra_flags or []), "-I", INCLUDE, "-I", CSRC]
    objs = [os.path.join(objdir, os.path.basename(src) + ".o") for src in SOURCES]
    jobs = [[hipcc(), *flags, "-c", src, "-o", obj] for src, obj in zip(SOURCES, objs)]
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "0") or 0) or (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            f.result()
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
