import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libssla_amd.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")


def assert_close(actual, ref, rtol, name="", atol_scale=None, ratio_mode=False):
    """Elementwise |a - b| <= rtol * |b| + atol with atol = rtol * rms(ref)
    (a bare rtol is ill-posed near zero), plus RMSE/RMS(ref) <= rtol.

    ratio_mode (bf16/fp16 GLA outputs): the bar is the reference's own
    error ratio RMSE/RMS(ref) <= rtol (get_err_ratio, reference
    utils/ela_utils.py:67-70), with every element still inside
    rtol * |b| + 10 * rtol * rms(ref) -- bf16 operand rounding puts a few
    elements of a 16M-element output several sigma out, as it does for the
    reference's own bf16 path."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(ref, dtype=np.float64)
    assert a.shape == b.shape, f"{name}: shape {a.shape} != {b.shape}"
    assert np.isfinite(a).all(), f"{name}: non-finite values"
    rms = float(np.sqrt(np.mean(b * b))) if b.size else 0.0
    atol = rtol * rms if atol_scale is None else atol_scale
    if ratio_mode:
        atol = 10 * rtol * rms
    err = np.abs(a - b)
    bad = err > rtol * np.abs(b) + atol
    ratio = float(np.sqrt(np.mean(err * err)) / (rms + 1e-30)) if b.size else 0.0
    assert not bad.any(), (f"{name}: {int(bad.sum())}/{bad.size} elements outside rtol={rtol} "
                           f"atol={atol:.3g}; max err {err.max():.3g}, rms ratio {ratio:.3g}")
    assert ratio <= rtol, f"{name}: RMSE/RMS {ratio:.3g} > {rtol}"
    return ratio
