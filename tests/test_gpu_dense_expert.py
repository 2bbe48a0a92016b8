"""The dense-expert decode branch on the GPU (`TPU_MOE_DENSE_EXPERT_THRESHOLD`,
`layers/core/fused_moe_gmm.py:669-686` -> `kernels/experimental/
moe_dense_expert.py`), on the reference test's fixture and routing cases
(`tests/kernels/experimental/test_moe_dense_expert.py`), with its
expert-parallel offset removed (ids outside the four local experts are -1).

Outputs are held to the north star's bar against the f32-accumulated oracle
of the same recipe (format ``fp8`` with the branch's zero-coefficient mask),
and by cosine to the dense-expert oracle as written (bf16 accumulator)."""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows
from oracle import codecs, moe as omoe
from test_oracle_moe import _dense_expert_fixture, dense_expert_case

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _weights(dev, w13, s13, w2, s2):
    f8 = torch.float8_e4m3fn
    return (_t(w13, dev).view(f8), _t(w2, dev).view(f8), _t(s13, dev), _t(s2, dev))


def _run(dev, monkeypatch, threshold, x, w, ids, weights, layout="package"):
    from qmoe.layers.fused_moe import fused_moe_gmm

    monkeypatch.setenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", str(threshold))
    w1, w2, s1, s2 = weights
    if layout == "reference":  # K-major weights, [E, 1, 1, N] scales
        w1, w2 = w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
        s1, s2 = s1[:, None, None, :].contiguous(), s2[:, None, None, :].contiguous()
    out = fused_moe_gmm(_t(x, dev, torch.bfloat16), w1, w2, s1, s2, None, None,
                        _t(w, dev, torch.bfloat16), _t(ids, dev), None, ids.shape[1], "silu")
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _cosine(a, b):
    return float(np.sum(a.astype(np.float64) * b) / (np.linalg.norm(a) * np.linalg.norm(b)))


@pytest.mark.parametrize("i", [512, 640])
@pytest.mark.parametrize("case", ["mixed", "single", "three", "duplicate", "empty", "zero"])
def test_dense_expert_cases(dev, monkeypatch, case, i):
    """`test_moe_dense_expert.py:40-120`: every routing case through the
    op; no active route gives exactly 0."""
    print(f"dense expert case={case} i={i}", flush=True)
    x, w13, s13, w2, s2 = _dense_expert_fixture(i)
    ids, w = dense_expert_case(case)
    got = _run(dev, monkeypatch, 1024, x, w, ids, _weights(dev, w13, s13, w2, s2))
    assert np.isfinite(got).all()
    if case in ("empty", "zero"):
        assert np.array_equal(got, np.zeros_like(got))
        return
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("fp8", w13, s13, w2, s2), w, ids, "silu",
                               skip_padded_tokens=True)
    assert_close_rows(got, ref, f"dense expert {case}")
    dense = omoe.dense_expert_moe(x, w13, s13, w2, s2, w, ids)
    assert _cosine(got, dense) >= 0.9995


def test_dense_expert_reference_layout_is_bit_identical(dev, monkeypatch):
    """The reference's runtime layout (`w1 [E, H, 2I]`, scales `[E, 1, 1, N]`,
    what its test passes) is admitted after the repack and gives the same
    bits as this package's layout."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    ids, w = dense_expert_case("mixed")
    wts = _weights(dev, w13, s13, w2, s2)
    a = _run(dev, monkeypatch, 1024, x, w, ids, wts)
    b = _run(dev, monkeypatch, 1024, x, w, ids, wts, layout="reference")
    assert np.array_equal(a, b)


def test_dense_expert_unaligned_tokens_keep_the_grouped_path(dev, monkeypatch):
    """`test_moe_dense_expert.py:152-179`: 15 tokens are not admitted; the
    output is bit-identical to the threshold-0 run."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    x = x[:15]
    ids, w = np.zeros((15, 1), np.int32), np.ones((15, 1), np.float32)
    wts = _weights(dev, w13, s13, w2, s2)
    a = _run(dev, monkeypatch, 0, x, w, ids, wts)
    b = _run(dev, monkeypatch, 1024, x, w, ids, wts)
    assert np.array_equal(a, b)


def test_dense_expert_nonfinite_expert_stays_with_its_tokens(dev, monkeypatch):
    """`test_moe_dense_expert.py:281-304`: expert 3's gate_up codes are NaN;
    tokens routed to expert 0 are finite and within the bar, tokens routed
    to 3 are NaN. A zero-weight route to expert 3 beside a route to expert 0
    contributes exactly nothing (the branch's coefficient mask): the same
    bits as the route alone."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    w13 = w13.copy()
    w13[3] = 0x7F  # e4m3fn NaN
    wts = _weights(dev, w13, s13, w2, s2)
    ids = np.where(np.arange(16)[:, None] < 8, 0, 3).astype(np.int32)
    got = _run(dev, monkeypatch, 1024, x, np.ones((16, 1), np.float32), ids, wts)
    assert np.isnan(got[8:]).all()
    ref = omoe.dense_expert_moe(x[:8], w13, s13, w2, s2, np.ones((8, 1), np.float32), ids[:8])
    assert _cosine(got[:8], ref) >= 0.9995
    ref32, _, _ = omoe.fused_moe(x[:8], omoe.ExpertWeights("fp8", w13, s13, w2, s2),
                                 np.ones((8, 1), np.float32), ids[:8], "silu")
    assert_close_rows(got[:8], ref32, "dense expert, finite tokens")

    ids2 = np.tile(np.array([[0, 3]], np.int32), (16, 1))
    masked = _run(dev, monkeypatch, 1024, x, np.tile(np.array([[1.0, 0.0]], np.float32), (16, 1)), ids2, wts)
    alone = _run(dev, monkeypatch, 1024, x, np.ones((16, 1), np.float32), ids2[:, :1], wts)
    assert np.isfinite(masked).all() and np.array_equal(masked, alone)


def test_dense_expert_opposite_routes_cancel(dev, monkeypatch):
    """`moe_dense_expert.py:258-268`: a token's routes to one expert merge
    into one coefficient before the mask, so weights +w and -w on the NaN
    expert 3 beside a route to expert 0 give exactly the route to 0 alone
    (the grouped sum w*y + (-w)*y would be NaN)."""
    print("dense expert +w/-w on a NaN expert", flush=True)
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    w13 = w13.copy()
    w13[3] = 0x7F  # e4m3fn NaN
    wts = _weights(dev, w13, s13, w2, s2)
    ids3 = np.tile(np.array([[0, 3, 3]], np.int32), (16, 1))
    w3 = np.tile(np.array([[1.0, 0.375, -0.375]], np.float32), (16, 1))
    merged = _run(dev, monkeypatch, 1024, x, w3, ids3, wts)
    alone = _run(dev, monkeypatch, 1024, x, np.ones((16, 1), np.float32), ids3[:, :1], wts)
    assert np.isfinite(merged).all() and np.array_equal(merged, alone)
    # two routes to expert 0 (0.25 + 0.75) are the single route of weight 1
    ids0 = np.tile(np.array([[0, 0]], np.int32), (16, 1))
    w0 = np.tile(np.array([[0.25, 0.75]], np.float32), (16, 1))
    assert np.array_equal(_run(dev, monkeypatch, 1024, x, w0, ids0, wts), alone)
