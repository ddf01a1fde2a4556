"""Shared pytest setup.

Tests marked ``gpu`` run the HIP kernels on an MI355X; everything else runs on
the CPU (oracle pins, host logic, the C-ABI library's exports and validation).
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "flash-attention-from-scratch_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

# Tolerances of the north star: max-abs error of the fp16 output against the
# fp32 oracle on identical inputs.
TOL = {64: 2e-3, 128: 4e-3}


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs the HIP kernels on an MI355X (gfx950)")


def _have_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


def pytest_collection_modifyitems(config, items):
    if _have_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def ext():
    """The built torch extension (builds it in-tree if absent)."""
    import attnkernels
    return attnkernels.load_extension()


def max_err(out, ref):
    """Max |out - ref| in float64 for numpy/torch inputs."""
    def as_np(x):
        if hasattr(x, "detach"):
            x = x.detach().float().cpu().numpy()
        return np.asarray(x, dtype=np.float64)
    return float(np.abs(as_np(out) - as_np(ref)).max()) if np.size(as_np(out)) else 0.0
