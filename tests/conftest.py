import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def mc():
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a HIP device")
    return torch.device("cuda:0")


def rel_err(out, ref):
    """max|out - ref| / max|ref| (the tolerance measure of the parity bar)."""
    if hasattr(out, "detach"):
        out = out.detach().float().cpu().numpy()
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    den = np.abs(ref).max()
    num = np.abs(out - ref).max()
    return float(num / den) if den > 0 else float(num)


def to_np(t):
    return t.detach().float().cpu().numpy()
