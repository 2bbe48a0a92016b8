"""The parity bars themselves (CPU): the same-codes bar of the GEMM tests
accepts the f32 summation-order differences it is meant to accept and fails
on planted mistakes of the kind it must catch (a 1% scale error, a dropped
bias, one wrong output)."""

import numpy as np
import pytest

from conftest import assert_close_rows, assert_close_same_codes, bf16_ulp
from oracle import codecs, linear, quant


def _case(seed=0, M=16, K=1024, N=256):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    ref, xq, sx = linear.w8a8_per_channel(x, wq, ws, "fp8")
    return ref, xq, sx, wq, ws


def test_bf16_ulp_values():
    assert bf16_ulp(1.0) == 2.0 ** -7
    assert bf16_ulp(1.99) == 2.0 ** -7
    assert bf16_ulp(2.0) == 2.0 ** -6
    assert bf16_ulp(-0.75) == 2.0 ** -8
    assert bf16_ulp(0.0) == 2.0 ** -133


def test_same_codes_bar_accepts_summation_order():
    """The same codes summed in f64 (another order, exact) and rounded as the
    kernel does pass the bar."""
    ref, xq, sx, wq, ws = _case()
    acc = codecs.e4m3_decode(xq).astype(np.float64) @ codecs.e4m3_decode(wq).astype(np.float64).T
    other = codecs.bf16_round(((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * ws[None, :]))
    assert_close_same_codes(other, ref, "f64 order")


@pytest.mark.parametrize("plant", ["scale_1pct", "bias", "one_output", "column_scale"])
def test_same_codes_bar_fails_planted_mistakes(plant):
    ref, _, _, _, ws = _case(1)
    bad = ref.copy()
    if plant == "scale_1pct":
        bad = codecs.bf16_round(ref * np.float32(1.01))
    elif plant == "bias":
        bad = codecs.bf16_round(ref + np.float32(0.05) * np.abs(ref).max())
    elif plant == "one_output":
        bad[3, 17] = codecs.bf16_round(np.float32(ref[3, 17] * 1.05 + 0.01))
    else:
        bad[:, 40] = codecs.bf16_round(ref[:, 40] * np.float32(1.02))
    with pytest.raises(AssertionError):
        assert_close_same_codes(bad, ref, plant)


def test_row_bar_is_the_north_star_tolerance():
    """max |err| <= 2e-2 * ||row||_inf and cosine >= 0.9995: a 3% row error
    fails, a 1% one passes."""
    ref, *_ = _case(2)
    assert_close_rows(ref * np.float32(1.01), ref, "1%")
    with pytest.raises(AssertionError):
        assert_close_rows(ref * np.float32(1.03), ref, "3%")
