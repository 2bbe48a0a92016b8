"""Pins the oracle's quantizers (CPU).

Known answers: `tests/layers/core/test_quantization_int_rounding.py` and
`test_quantization_zero_blocks.py` of the reference. The runtime quantizer's
float32 (fp8) and bf16 (int8) arithmetic is checked against torch doing the
same operations in those dtypes (torch's bf16 division is the correctly
rounded quotient, as JAX's is).
"""

import numpy as np
import pytest
import torch

from oracle import codecs, quant


def test_half_lsb_ties_round_half_to_even():
    # test_quantization_int_rounding.py:53-76
    t = np.float32([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 63.5]])
    q, s = quant.quantize_tensor(t, "int8")
    assert s[0] == 1.0
    np.testing.assert_array_equal(q, [[127, 0, 2, 2, 0, -2, -2, 64]])


def test_float_targets_keep_the_sub_unit_grid():
    # test_quantization_int_rounding.py:109-118
    t = np.float32([[448.0, 0.5, 1.5, 2.5]])
    q, s = quant.quantize_tensor(t, "fp8")
    assert s[0] == 1.0
    np.testing.assert_array_equal(codecs.e4m3_decode(q), t)


def test_zero_rows_stay_zero():
    # test_quantization_zero_blocks.py:25-54
    t = np.float32([[0, 0, 0, 0], [1, -2, 3, -4]])
    q, s = quant.quantize_tensor(t, "fp8")
    assert s[0] == 0.0
    np.testing.assert_array_equal(codecs.e4m3_decode(q[0]), 0)
    assert np.isfinite(codecs.e4m3_decode(q)).all()


def test_reciprocal_multiply_scale_rounding():
    # test_quantization_zero_blocks.py:57-68: scale == amax * f32(1/448) exactly
    t = np.float32([[0.0010000200709328055]])
    _, s = quant.quantize_tensor(t, "fp8")
    assert s[0] == np.float32(0.0010000200709328055) * np.float32(1.0 / 448.0)


def test_integer_error_matches_uniform_half_lsb_bound():
    # test_quantization_int_rounding.py:96-106
    t = np.random.default_rng(0).standard_normal((4, 8192)).astype(np.float32)
    q, s = quant.quantize_tensor(t, "int8")
    err = (t - q.astype(np.float32) * s[:, None]) / s[:, None]
    assert np.abs(err).max() <= 0.5 + 1e-3
    assert abs(err.mean()) < 0.01
    assert err.std() == pytest.approx(12 ** -0.5, rel=0.05)


def test_load_time_fp8_matches_torch_restatement():
    # same operations as `layers/core/quantization.py:273-315`, in torch
    w = torch.randn(64, 512, generator=torch.Generator().manual_seed(5)) * 0.02
    scale = w.abs().amax(-1, keepdim=True) * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    inv = torch.where(scale == 0, torch.zeros_like(scale), 1.0 / scale)
    qt = torch.clamp(w * inv, -448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    q, s = quant.quantize_tensor(w.numpy(), "fp8")
    np.testing.assert_array_equal(q, qt)
    np.testing.assert_array_equal(s, scale[:, 0].numpy())


def test_runtime_fp8_matches_f32_torch():
    # util.py:303-318 with a float8 target: float32 division, clip, RNE cast
    x = (torch.randn(16, 1024, generator=torch.Generator().manual_seed(2)) * 3).to(torch.bfloat16).float()
    x[3] = 0.0
    amax = x.abs().amax(-1, keepdim=True)
    sc = amax / 448.0
    sc = torch.where(sc == 0, torch.ones_like(sc), sc)
    qt = torch.clamp(x / sc, -448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    q, s = quant.quantize_act(x.numpy(), "fp8")
    np.testing.assert_array_equal(q, qt)
    np.testing.assert_array_equal(s, sc[:, 0].numpy())
    assert s[3] == 1.0


def test_runtime_int8_matches_bf16_torch():
    # util.py:303-318 with an int8 target: every op in bf16 (weak-typed 127)
    x = (torch.randn(16, 1024, generator=torch.Generator().manual_seed(3)) * 2).to(torch.bfloat16)
    amax = x.abs().amax(-1, keepdim=True)
    sc = amax / 127  # bf16 tensor / python int -> bf16
    assert sc.dtype == torch.bfloat16
    sc = torch.where(sc == 0, torch.ones_like(sc), sc)
    qt = torch.round(x / sc).float().clamp(-128, 127).to(torch.int8).numpy()
    q, s = quant.quantize_act(x.float().numpy(), "int8")
    np.testing.assert_array_equal(q, qt)
    np.testing.assert_array_equal(s, sc[:, 0].float().numpy())


def test_runtime_block_scales_are_per_128():
    x = codecs.bf16_round(np.random.default_rng(9).standard_normal((3, 512)).astype(np.float32))
    q, s = quant.quantize_act(x, "fp8", block=128)
    assert s.shape == (3, 4)
    for b in range(4):
        qb, sb = quant.quantize_act(x[:, b * 128:(b + 1) * 128], "fp8")
        np.testing.assert_array_equal(q[:, b * 128:(b + 1) * 128], qb)
        np.testing.assert_array_equal(s[:, b], sb)


def test_tile_quant_roundtrip_error_bound():
    w = np.random.default_rng(4).standard_normal((256, 384)).astype(np.float32) * 0.02
    c, s = quant.quantize_fp8_tiles(w)
    assert s.shape == (2, 3)
    d = quant.dequant_tiles(c, s)
    rel = np.abs(d - w) / np.repeat(np.repeat(s, 128, 0), 128, 1)
    assert rel.max() <= 16.0 + 1e-3  # half an ulp of 448's binade in scale units
