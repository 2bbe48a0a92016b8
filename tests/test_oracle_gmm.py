"""Pins of the oracle's grouped-matmul regimes (CPU): the per-(row, 512)
bf16-arithmetic activation quant, the per-channel quantized-lhs GEMM and the
bf16-dequantized block-FP8 GEMM (`kernels/megablox/gmm_v2.py:452-462,
500-548`).

Each pin is computed independently of the oracle's formulas: hand-worked
bf16 / e4m3 values, the already pinned per-128 runtime quantizer on inputs
where the two recipes must agree, and a dequantize-then-matmul computation
in float64."""

import numpy as np
import pytest

from oracle import codecs, linear, quant


def _bf(v):
    return codecs.bf16_round(np.asarray(v, np.float32))


def test_gmm_fp8_known_answers():
    """absmax 448 -> scale 1, codes are the e4m3 of x; absmax 1 -> scale
    bf16(1/448) = 146/128 * 2^-9 and inv bf16(448.877) = 448, so 0.1 (bf16
    0.10009765625) -> bf16(44.84375) = 44.75 -> e4m3 44 (0x63)."""
    x = np.zeros((2, 512), np.float32)
    x[0, :5] = [448.0, 1.0, -0.5, 3.0, 0.0]
    x[1, :3] = [1.0, 0.1, -1.0]
    q, s = quant.quantize_gmm_lhs(_bf(x), "fp8")
    assert s.shape == (2, 1)
    assert s[0, 0] == 1.0
    assert s[1, 0] == np.float32(146 / 128 * 2.0 ** -9)
    assert q[0, :5].tolist() == [0x7E, 0x38, 0xB0, 0x44, 0x00]
    assert q[1, :3].tolist() == [0x7E, 0x63, 0xFE]


def test_gmm_int8_truncates_toward_zero():
    """The int8 codes are `.astype(int8)` of the bf16 product: truncation,
    not rounding (scale bf16(127/127) = 1)."""
    x = np.zeros((1, 512), np.float32)
    x[0, :8] = [127.0, 3.75, -3.75, 0.5, -0.5, 63.5, -63.5, 1.99]
    q, s = quant.quantize_gmm_lhs(_bf(x), "int8")
    assert s[0, 0] == 1.0
    assert q[0, :8].tolist() == [127, 3, -3, 0, 0, 63, -63, 1]
    # absmax 254 -> scale 2, inv 0.5: 7 -> 3.5 -> 3
    x[0, 0] = 254.0
    x[0, 1] = 7.0
    q, s = quant.quantize_gmm_lhs(_bf(x), "int8")
    assert s[0, 0] == 2.0 and q[0, 1] == 3


def test_gmm_blocks_start_at_column_zero_and_zero_blocks_keep_scale_zero():
    """Blocks of 512 from column 0, the last one partial (K = 1152: 512, 512,
    128); an all-zero block keeps scale 0 and codes 0."""
    rng = np.random.default_rng(0)
    x = _bf(rng.standard_normal((3, 1152)).astype(np.float32))
    x[:, 512:1024] = 0.0
    x[1, 1100] = 1000.0  # only the partial block sees it
    q, s = quant.quantize_gmm_lhs(x, "fp8")
    assert s.shape == (3, 3)
    assert (s[:, 1] == 0).all() and (q[:, 512:1024] == 0).all()
    assert s[1, 2] == _bf(np.float32(1000.0) / np.float32(448.0))
    assert s[1, 0] == s[1, 0] and s[1, 0] < 1.0  # block 0 unaffected by the outlier


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_gmm_agrees_with_runtime_quant_at_power_of_two_scales(qdtype):
    """When every 128-column block of a 512-column block holds the same
    absmax qmax * 2^j, both recipes have scale 2^j exactly; the fp8 codes
    then equal the pinned per-128 runtime quantizer's (e4m3 RNE of x * 2^-j),
    and the int8 codes are its codes truncated instead of rounded."""
    rng = np.random.default_rng(1)
    qmax = 448.0 if qdtype == "fp8" else 127.0
    m, k = 6, 2048
    x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    for r in range(m):
        for b in range(k // 512):
            j = rng.integers(-6, 4)
            sl = slice(b * 512, (b + 1) * 512)
            x[r, sl] *= qmax * 2.0 ** j
            x[r, b * 512:(b + 1) * 512:128] = qmax * 2.0 ** j  # the max in every 128-block
    x = _bf(x)
    q, s = quant.quantize_gmm_lhs(x, qdtype)
    if qdtype == "fp8":
        q_rt, s_rt = quant.quantize_act(x, "fp8", block=128)
        np.testing.assert_array_equal(np.repeat(s, 4, axis=1), s_rt)
        np.testing.assert_array_equal(q, q_rt)
    else:
        sc = np.repeat(s, 512, axis=1)
        np.testing.assert_array_equal(q, np.trunc(x / sc).astype(np.int8))
        assert (np.trunc(x / sc) != np.rint(x / sc)).any()  # the truncation matters here


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("K", [1024, 1152, 2048])
def test_gmm_gemm_equals_dequantize_then_matmul(qdtype, K):
    """w8a8_gmm (block dots x activation scale, summed, x weight scale) equals
    the float64 matmul of the dequantized operands (codes times their block /
    channel scales) to float32 rounding: each 512-column block carries its
    own activation scale, so a block-index slip fails this."""
    rng = np.random.default_rng(K)
    M, N = 9, 70
    x = _bf(rng.standard_normal((M, K)).astype(np.float32) * rng.uniform(0.1, 10, (M, 1)))
    x[:, 512:640] *= 40.0  # blocks with very different scales
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    y, xq, xs = linear.w8a8_gmm(x, wq, ws, qdtype, round_out=False)
    xd = quant.dequant_codes(xq, qdtype).astype(np.float64) * np.repeat(xs, 512, axis=1)[:, :K]
    wd = quant.dequant_codes(wq, qdtype).astype(np.float64) * ws[:, None].astype(np.float64)
    ref = xd @ wd.T
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=2e-6 * np.abs(ref).max())


def test_gmm_bf16_accumulation_is_within_the_parity_bar():
    """The reference's bf16 accumulator stays within the north-star bar of
    the float32-accumulated form on config-like data (K 7168)."""
    from conftest import assert_close_rows

    rng = np.random.default_rng(3)
    M, K, N = 8, 7168, 256
    x = _bf(rng.standard_normal((M, K)).astype(np.float32))
    wq, ws = quant.quantize_tensor((rng.standard_normal((N, K)) * 0.02).astype(np.float32), "fp8")
    y32, _, _ = linear.w8a8_gmm(x, wq, ws, "fp8")
    y16 = linear.w8a8_gmm_bf16acc(x, wq, ws, "fp8")
    assert_close_rows(y32, y16, "bf16 vs f32 accumulation")
    assert not np.array_equal(y32, y16)  # the accumulators do differ


def test_w8a16_blockwise_known_answer_and_rounding():
    """Each weight is bf16(code * bf16(scale)): code 1.5 (0x3C) x scale
    1.0078125 -> 1.51171875 -> bf16 1.515625; a one-hot activation reads it
    back. Uniform block scales equal the per-channel W8A16 result."""
    wq = np.full((4, 256), 0x3C, np.uint8)  # e4m3 1.5
    sb = np.full((4, 2), 1.0078125, np.float32)
    x = np.zeros((2, 256), np.float32)
    x[0, 3] = 1.0
    x[1, 200] = 2.0
    y = linear.w8a16_blockwise(x, wq, sb)
    assert (y[0] == 1.515625).all() and (y[1] == 3.03125).all()
    # scale rounded to bf16 first: 1.00390625 (a bf16 tie) -> 1.0
    sb2 = np.full((4, 2), 1.00390625, np.float32)
    assert (linear.w8a16_blockwise(x, wq, sb2)[0] == 1.5).all()
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    ws = _bf(ws)  # bf16-valued channel scales: then the bf16 dequantization is the same per block
    xr = _bf(rng.standard_normal((5, 512)).astype(np.float32))
    blk = linear.w8a16_blockwise(xr, wq, np.repeat(ws[:, None], 4, axis=1))
    deq = _bf(codecs.e4m3_decode(wq) * ws[:, None])
    np.testing.assert_array_equal(blk, linear.w16a16(xr, deq))
