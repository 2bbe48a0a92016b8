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


# ---------------------------------------------------------------- MX activations


def _torch_ue8m0_exponent(scale):
    """The reference's exponent rule executed literally in torch f32
    (`layers/core/quantization.py:285-298`: ceil(log2), repair, clamp)."""
    s = torch.from_numpy(np.asarray(scale, np.float32))
    e = torch.ceil(torch.log2(s))
    e = torch.where(torch.exp2(e) < s, e + 1, e).clamp(-127, 127)
    return e.to(torch.int64).numpy()


def test_mx_exponent_matches_log2_rule_and_is_minimal():
    rng = np.random.default_rng(3)
    amax = np.concatenate([
        np.abs(rng.standard_normal(4000)).astype(np.float32) * np.float32(2.0) ** rng.integers(-40, 40, 4000),
        (6.0 * np.float32(2.0) ** np.arange(-60, 60)).astype(np.float32),           # exact powers after /6
        np.nextafter((6.0 * np.float32(2.0) ** np.arange(-60, 60)).astype(np.float32), np.float32(np.inf)),
        np.float32([0.0, 1e-45, 1e-40, 3e38]),
    ]).astype(np.float32)
    scale = (amax * np.float32(1.0 / 6.0)).astype(np.float32)
    e = quant.e8m0_exponent_ceil(scale)
    np.testing.assert_array_equal(e, _torch_ue8m0_exponent(scale))
    # 2**e covers the scale and 2**(e-1) does not (inside the clamp range)
    p = np.ldexp(1.0, e)
    assert (p >= scale).all()
    inner = e > -127
    assert (np.ldexp(1.0, e[inner] - 1) < scale[inner]).all()


def test_mx_known_answers():
    # amax 6 -> scale 1 -> byte 127; edge values take the lower code
    x = np.zeros((1, 32), np.float32)
    x[0, :8] = [6.0, 3.0, -1.25, 0.3, 0.75, -5.0, 5.01, -0.0]
    q, s = quant.quantize_mx_fp4(x)
    assert s.tolist() == [[127]]
    nib = codecs.unpack_fp4(q)[0, :8]
    # 6 -> 7, 3 -> 5, -1.25 -> -(1.0), 0.3 -> 0.5, 0.75 -> 0.5, -5 -> -(4.0), 5.01 -> 6, -0 -> +0
    assert nib.tolist() == [7, 5, 8 | 2, 1, 1, 8 | 6, 7, 0]
    # amax 12 -> scale 2 -> byte 128; amax 6.5 -> scale > 1 -> byte 128 as well
    for amax, byte in ((12.0, 128), (6.5, 128), (3.0, 126), (0.0, 0)):
        x = np.zeros((1, 32), np.float32)
        x[0, 5] = amax
        q, s = quant.quantize_mx_fp4(x)
        assert s[0, 0] == byte, (amax, s)
    # zero padding to the requested width
    q, s = quant.quantize_mx_fp4(np.ones((2, 32), np.float32), k_pad=96)
    assert q.shape == (2, 48) and s.shape == (2, 3)
    assert (q[:, 16:] == 0).all() and (s[:, 1:] == 0).all()


def test_mx_encoder_is_nearest_with_ties_down_and_matches_bucketize():
    v = np.concatenate([np.linspace(-7, 7, 20001), quant.FP4_EDGES, -quant.FP4_EDGES]).astype(np.float32)
    c = quant.fp4_encode_bucket(v)
    mags = np.float32([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    dist = np.abs(np.abs(v)[:, None] - mags[None, :])
    got = np.abs(codecs.fp4_decode(c))
    best = dist.min(axis=1)
    assert np.allclose(np.abs(np.abs(v) - got), best, rtol=0, atol=0)
    lower = mags[np.argmin(dist, axis=1)]  # argmin takes the first (lower) of two equal distances
    np.testing.assert_array_equal(got, lower)
    # the reference's own call, torch.bucketize(|v|, edges) | sign
    t = torch.from_numpy(v)
    ref = torch.bucketize(t.abs(), torch.from_numpy(quant.FP4_EDGES)).to(torch.uint8)
    ref = ref | torch.where(t < 0, 8, 0).to(torch.uint8)
    np.testing.assert_array_equal(c, ref.numpy())


def test_mx_reproduces_representable_values_and_error_bound():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((16, 256)) * np.float32(2.0) ** rng.integers(-6, 6, (16, 1))).astype(np.float32)
    q, s = quant.quantize_mx_fp4(x)
    d = codecs.dequant_mxfp4(q, s)
    # error within half the widest e2m1 gap (1.0 at the top) times the block scale
    blk = np.repeat(codecs.e8m0_decode(s), 32, axis=1)
    assert (np.abs(d - x) <= blk).all()
    # MX values quantize to themselves (a block whose top code is 3.0 moves
    # one octave down and doubles its codes: same values)
    q2, s2 = quant.quantize_mx_fp4(d)
    np.testing.assert_array_equal(codecs.dequant_mxfp4(q2, s2), d)


def test_mx_quant_non_finite_blocks_are_nan_blocks():
    """The build's definition for inf / NaN inside a 32-value block (the
    reference's rule has none): codes 0, byte 255 (e8m0 NaN), so the block
    decodes to NaN; the row's finite blocks quantize exactly as they do with
    the bad block replaced by zeros."""
    from oracle import codecs

    rng = np.random.default_rng(3)
    x = codecs.bf16_round(rng.standard_normal((2, 128)).astype(np.float32))
    y = x.copy()
    y[0, 40] = np.inf
    y[1, 127] = np.nan
    q, s = quant.quantize_mx_fp4(y)
    z = x.copy()
    z[0, 32:64] = 0.0
    z[1, 96:128] = 0.0
    qz, sz = quant.quantize_mx_fp4(z)
    assert s[0, 1] == 255 and s[1, 3] == 255
    assert (q[0, 16:32] == 0).all() and (q[1, 48:64] == 0).all()
    keep = np.ones_like(s, bool)
    keep[0, 1] = keep[1, 3] = False
    np.testing.assert_array_equal(s[keep], sz[keep])
    np.testing.assert_array_equal(q[:, :16], qz[:, :16])
    with np.errstate(invalid="ignore"):
        d = codecs.dequant_mxfp4(q, s)
    assert np.isnan(d[0, 32:64]).all() and np.isnan(d[1, 96:]).all()
    assert np.isfinite(d[0, :32]).all() and np.isfinite(d[1, :96]).all()


def test_e5m2_quantizers():
    """float8_e5m2 targets: the load-time quantizer's codes are torch's
    e5m2 cast of the clipped reciprocal-scaled values (scale = amax *
    f32(1/57344)); the runtime quantizer divides by amax / 57344 in f32;
    both read back within the e5m2 quantum (2 mantissa bits: 12.5 % of the
    binade)."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((6, 256)) * 0.02).astype(np.float32)
    q, s = quant.quantize_tensor(w, "e5m2")
    scale = (np.abs(w).max(axis=-1) * np.float32(1.0 / 57344.0)).astype(np.float32)
    np.testing.assert_array_equal(s, scale)
    t = np.clip(w * (np.float32(1.0) / scale)[:, None], -57344, 57344).astype(np.float32)
    np.testing.assert_array_equal(q, torch.from_numpy(t).to(torch.float8_e5m2).view(torch.uint8).numpy())
    back = codecs.e5m2_decode(q) * s[:, None]
    assert np.all(np.abs(back - w) <= 0.125 * np.abs(w) + 1e-30 + 2.0 ** -16 * s[:, None])
    x = codecs.bf16_round(rng.standard_normal((3, 128)).astype(np.float32))
    xq, xs = quant.quantize_act(x, "e5m2")
    sx = (np.abs(x).max(axis=-1) / np.float32(57344.0)).astype(np.float32)
    np.testing.assert_array_equal(xs, sx)
    ref = torch.from_numpy(np.clip(x / sx[:, None], -57344, 57344).astype(np.float32)).to(torch.float8_e5m2)
    np.testing.assert_array_equal(xq, ref.view(torch.uint8).numpy())
    assert codecs.e5m2_decode(xq).max() == 57344.0  # the row maximum maps to the e5m2 maximum
