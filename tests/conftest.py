import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# north-star gates
ATOL_F16 = 1e-2
RTOL_F16 = 2e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


def assert_close(got, ref, atol=ATOL_F16, rtol=RTOL_F16, what=""):
    """|got - ref| <= atol + rtol*|ref| elementwise, non-finite values fail."""
    g = got.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert g.shape == r.shape, f"{what}: shape {tuple(g.shape)} != {tuple(r.shape)}"
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    d = (g - r).abs()
    bad = d > atol + rtol * r.abs()
    if bad.any():
        i = tuple(int(v) for v in bad.nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} outside atol={atol} rtol={rtol}; "
            f"max|d|={float(d.max()):.4g}; first {i}: got {float(g[i]):.6g} ref {float(r[i]):.6g}")


@pytest.fixture
def rng():
    return np.random.default_rng(20260901)
