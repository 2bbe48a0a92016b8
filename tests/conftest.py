import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "vllm-torchtpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def assert_close_rows(got, ref, what="", rel=2e-2, cos_min=0.9995):
    """The parity bar for bf16 outputs: per row max |err| <= rel * max|ref row|
    and cosine >= cos_min over the whole tensor (fp32-accumulated oracle)."""
    got = np.asarray(got, np.float64).reshape(-1, np.asarray(got).shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, np.asarray(ref).shape[-1])
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref).max(axis=-1)
    lim = rel * np.maximum(np.abs(ref).max(axis=-1), 1e-12)
    bad = np.nonzero(err > lim)[0]
    assert bad.size == 0, f"{what}: rows {bad[:8]} exceed tol: err {err[bad[:4]]} lim {lim[bad[:4]]}"
    den = np.linalg.norm(got) * np.linalg.norm(ref)
    if den > 0:
        cos = float((got * ref).sum() / den)
        assert cos >= cos_min, f"{what}: cosine {cos:.6f} < {cos_min}"
