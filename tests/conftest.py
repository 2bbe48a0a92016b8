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


def bf16_ulp(v):
    """The spacing of bf16 values at |v| (the smallest normal spacing below
    2**-126)."""
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def assert_close_same_codes(got, ref, what="", abs_rel=2.0 ** -12):
    """The parity bar when the kernel and the oracle multiply the same codes
    (FP8 / e2m1 / bf16 operands are exact in f32, so only the summation
    differs): each bf16 output is within one bf16 ulp of the oracle's bf16
    output, plus ``abs_rel`` times the row's max. The second term covers the
    sums of near-zero outputs: an MFMA adds its products in hardware that does
    not round like an f32 BLAS does (measured on MI355X: up to ~2^-15 of the
    row max at K = 4096, FP8 codes). A scale, bias or epilogue error of 1%
    or more fails it (tests/test_parity_bars.py plants such errors)."""
    got = np.asarray(got, np.float64).reshape(-1, np.asarray(got).shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, np.asarray(ref).shape[-1])
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    rowmax = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
    lim = bf16_ulp(np.maximum(np.abs(got), np.abs(ref))) + abs_rel * rowmax
    err = np.abs(got - ref)
    bad = np.argwhere(err > lim)
    assert bad.size == 0, (f"{what}: {len(bad)} outputs beyond 1 bf16 ulp, first at {bad[:4].tolist()}: "
                           f"got {got[tuple(bad[0])]} ref {ref[tuple(bad[0])]}")
