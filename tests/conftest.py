import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def normwise_err(got, ref) -> float:
    """max|got - ref| / max|ref| -- the parity metric for attention outputs.

    Per-element relative error is ill-conditioned here: outputs are sums of
    many signed terms and some land near zero, where independent fp32
    summation orders differ by ~sqrt(n)*eps*|typical output|.  The reference's
    own check uses an absolute bound for the same reason (bench/bench.cc:214-216).
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = float(np.max(np.abs(ref)))
    if scale == 0.0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - ref)) / scale)


@pytest.fixture(scope="session")
def gpu():
    """A usable GPU with the built library, or a loud failure (never a fallback)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import molot_amd

    molot_amd.load()  # raises if the native library is missing
    return torch.device("cuda:0")
