"""Pins of the dense linear references in `oracle/linear.py` (CPU).

Each expected value here is fixed without the oracle's own formula:

* the reference's known answer for the FP8 linear method (ones weights,
  unit scales, ones activations -> ``in_dim``; `tests/layers/adapter/
  quantization/test_fp8.py:1208-1238`), applied to every dense recipe;
* hand-built operands whose quantization is exact (power-of-two scales,
  small integer codes), so the result is an integer sum computed here in
  int64 / float64;
* structural identities: uniform block scales make the blockwise recipe the
  per-channel one, a one-hot activation reads a dequantized weight back,
  bias and column permutations commute with the matmul.

A plausible mistake in the oracle -- a transposed scale, a dropped block
scale, a block index off by one, a missing bias, the wrong axis of the
activation scale -- fails at least one of these.
"""

import numpy as np
import pytest
import torch

from oracle import codecs, linear, quant


def _bf(v):
    return codecs.bf16_round(np.asarray(v, np.float32))


def _torch_bf16(v64):
    """float64 -> bf16 value (as float32) through torch's own cast."""
    return torch.from_numpy(np.asarray(v64, np.float64)).to(torch.bfloat16).float().numpy()


# ---------------------------------------------------------------------------
# the reference's known answer: ones x ones -> K
# ---------------------------------------------------------------------------

def _ones_case(k=128, n=64, m=4):
    x = np.ones((m, k), np.float32)
    one = codecs.e4m3_encode(np.ones((n, k), np.float32))
    return x, one


@pytest.mark.parametrize("k", [128, 512, 1024])
def test_ones_known_answer_every_dense_recipe(k):
    """`test_fp8.py:1208-1238`: an all-ones e4m3 weight with unit scales
    times ones gives ``in_dim`` (128 there; the same holds for any K whose
    sum is a bf16 value), within the reference's 1% -- here exactly, since
    the only rounding is the activation scale's, far below a bf16 ulp."""
    x, w8 = _ones_case(k)
    n = w8.shape[0]
    ones_n = np.ones(n, np.float32)
    outs = {
        "w8a8 fp8": linear.w8a8_per_channel(x, w8, ones_n, "fp8")[0],
        "w8a8 int8": linear.w8a8_per_channel(x, np.ones((n, k), np.int8), ones_n, "int8")[0],
        "w8a16": linear.w8a16_per_channel(x, w8, ones_n),
        "blockwise": linear.w8a8_blockwise(x, w8, np.ones((n, k // 128), np.float32))[0],
        "gmm fp8": linear.w8a8_gmm(x, w8, ones_n, "fp8")[0],
        "gmm int8": linear.w8a8_gmm(x, np.ones((n, k), np.int8), ones_n, "int8")[0],
        "gmm bf16 acc": linear.w8a8_gmm_bf16acc(x, w8, ones_n, "fp8"),
        "w8a16 blocks": linear.w8a16_blockwise(x, w8, np.ones((n, k // 128), np.float32)),
        "w16a16": linear.w16a16(x, np.ones((n, k), np.float32)),
    }
    for name, y in outs.items():
        assert y.shape == (x.shape[0], n), name
        np.testing.assert_array_equal(y, np.full_like(y, float(k)), err_msg=name)


def test_ones_known_answer_w4a16_kinds():
    """The same known answer through the 4-bit weight formats: e2m1 1.0 is
    nibble 0x2, e8m0 127 is 2^0; NVFP4 fused scale 1.0; int4 +1 with scale 1."""
    k, n, m = 256, 32, 3
    x = np.ones((m, k), np.float32)
    packed = codecs.pack_fp4(np.full((n, k), 0x2, np.uint8))
    y = linear.w4a16_mxfp4(x, packed, np.full((n, k // 32), 127, np.uint8))
    np.testing.assert_array_equal(y, np.full((m, n), float(k), np.float32))
    y = linear.w4a16_nvfp4(x, packed, np.ones((n, k // 16), np.float32))
    np.testing.assert_array_equal(y, np.full((m, n), float(k), np.float32))
    carriers = codecs.int4_pack(np.ones((n, k), np.int8))
    y = linear.w4a16_int4(x, carriers, np.ones((n, k // 128), np.float32))
    np.testing.assert_array_equal(y, np.full((m, n), float(k), np.float32))


# ---------------------------------------------------------------------------
# exact integer cases with power-of-two scales
# ---------------------------------------------------------------------------

def _pow2_rows(rng, m, k, qmax, block=None, small=8):
    """Activations whose quantization is exact: each (row, block) holds
    small integers times 2^j plus one element +-qmax * 2^j (its absmax), so
    the scale is 2^j exactly and the codes are the integers. Returns
    (x, integer codes, exponents [m, nblocks])."""
    block = block or k
    nb = k // block
    codes = rng.integers(-small, small + 1, (m, k)).astype(np.int64)
    j = rng.integers(-5, 4, (m, nb))
    for r in range(m):
        for b in range(nb):
            codes[r, b * block + rng.integers(0, block)] = qmax * (1 if rng.random() < 0.5 else -1)
    x = codes.astype(np.float64) * np.repeat(2.0 ** j, block, axis=1)
    return x.astype(np.float32), codes, j


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_per_channel_exact_integer_sums(qdtype):
    """Per-token activation scale 2^j, weight codes small integers with
    per-channel scales 2^i: the output is bf16(2^(i+j) * integer dot) --
    computed here in int64 and rounded by torch. A transposed or dropped
    scale changes the power of two."""
    rng = np.random.default_rng(11)
    m, k, n = 5, 256, 24
    qmax = 448 if qdtype == "fp8" else 127
    x, xc, j = _pow2_rows(rng, m, k, qmax)
    wc = rng.integers(-6, 7, (n, k)).astype(np.int64)
    wi = rng.integers(-4, 3, n)
    ws = (2.0 ** wi).astype(np.float32)
    wq = codecs.e4m3_encode(wc.astype(np.float32)) if qdtype == "fp8" else wc.astype(np.int8)
    y, xq, sx = linear.w8a8_per_channel(x, wq, ws, qdtype)
    np.testing.assert_array_equal(sx, (2.0 ** j[:, 0]).astype(np.float32))
    want = (xc @ wc.T).astype(np.float64) * 2.0 ** j[:, :1] * 2.0 ** wi[None, :]
    np.testing.assert_array_equal(y, _torch_bf16(want))
    # w8a16: bf16 x unquantized times the weight codes
    if qdtype == "fp8":
        xb = _bf(x)
        want16 = (xb.astype(np.float64) @ wc.T.astype(np.float64)) * 2.0 ** wi[None, :]
        np.testing.assert_array_equal(linear.w8a16_per_channel(xb, wq, ws), _torch_bf16(want16))


def test_blockwise_exact_integer_sums():
    """Per-(token, 128) activation scales 2^j[b] and per-(n, 128) weight
    scales 2^i[n, b], different for every block: the output is
    bf16(sum_b 2^(j[b] + i[n, b]) * integer block dot). An off-by-one block
    index or a transposed weight-scale table fails."""
    rng = np.random.default_rng(12)
    m, k, n = 4, 512, 16
    x, xc, j = _pow2_rows(rng, m, k, 448, block=128)
    wc = rng.integers(-6, 7, (n, k)).astype(np.int64)
    wi = rng.integers(-3, 3, (n, k // 128))
    wsb = (2.0 ** wi).astype(np.float32)
    y, xq, xs = linear.w8a8_blockwise(x, codecs.e4m3_encode(wc.astype(np.float32)), wsb)
    np.testing.assert_array_equal(xs, (2.0 ** j).astype(np.float32))
    want = np.zeros((m, n), np.float64)
    for b in range(k // 128):
        sl = slice(b * 128, (b + 1) * 128)
        want += (xc[:, sl] @ wc[:, sl].T) * 2.0 ** j[:, b:b + 1] * 2.0 ** wi[None, :, b]
    np.testing.assert_array_equal(y, _torch_bf16(want))


def test_w8a16_blockwise_exact_integer_sums():
    """bf16 x times bf16(code * bf16(scale)) with power-of-two block scales:
    the weights are exact, so the output is bf16 of the float64 sum."""
    rng = np.random.default_rng(13)
    m, k, n = 3, 384, 20
    xb = _bf(rng.integers(-20, 21, (m, k)).astype(np.float32) * 0.25)
    wc = rng.integers(-6, 7, (n, k)).astype(np.int64)
    wi = rng.integers(-3, 3, (n, k // 128))
    y = linear.w8a16_blockwise(xb, codecs.e4m3_encode(wc.astype(np.float32)), (2.0 ** wi).astype(np.float32))
    wd = wc.astype(np.float64) * np.repeat(2.0 ** wi, 128, axis=1)
    np.testing.assert_array_equal(y, _torch_bf16(xb.astype(np.float64) @ wd.T))


def test_w4a16_exact_integer_sums():
    """MXFP4 codes {0, +-0.5 .. +-6} times e8m0 2^(s-127) per 32 columns,
    small-integer activations: the dequantized weights are exact and the
    sums are computed here in float64. Each 32-column block has its own
    exponent, so a scale read from the wrong block fails."""
    rng = np.random.default_rng(14)
    m, k, n = 4, 256, 12
    nib = rng.integers(0, 16, (n, k)).astype(np.uint8)
    e = rng.integers(124, 131, (n, k // 32)).astype(np.uint8)
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    wv = np.where(nib >= 8, -1.0, 1.0) * e2m1[nib & 7] * np.repeat(2.0 ** (e.astype(np.int64) - 127), 32, axis=1)
    x = rng.integers(-4, 5, (m, k)).astype(np.float32)
    bias = (rng.integers(-8, 9, n) * 0.5).astype(np.float32)
    y = linear.w4a16_mxfp4(x, codecs.pack_fp4(nib), e, bias=bias)
    np.testing.assert_array_equal(y, _torch_bf16(x.astype(np.float64) @ wv.T + bias))
    # int4 values -8..7 with power-of-two group scales (group 128)
    iv = rng.integers(-8, 8, (n, k)).astype(np.int8)
    gi = rng.integers(-3, 3, (n, k // 128))
    y = linear.w4a16_int4(x, codecs.int4_pack(iv), (2.0 ** gi).astype(np.float32), bias=bias)
    wd = iv.astype(np.float64) * np.repeat(2.0 ** gi, 128, axis=1)
    np.testing.assert_array_equal(y, _torch_bf16(x.astype(np.float64) @ wd.T + bias))


def test_nvfp4_one_hot_reads_back_the_dequantized_weight():
    """A one-hot activation row returns one dequantized weight column; with
    power-of-two fused scales that is e2m1 * scale exactly."""
    rng = np.random.default_rng(15)
    k, n = 128, 16
    nib = rng.integers(0, 16, (n, k)).astype(np.uint8)
    sc = (2.0 ** rng.integers(-4, 4, (n, k // 16))).astype(np.float32)
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    wv = np.where(nib >= 8, -1.0, 1.0) * e2m1[nib & 7] * np.repeat(sc, 16, axis=1)
    cols = [0, 15, 16, 77, 127]
    x = np.zeros((len(cols), k), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = linear.w4a16_nvfp4(x, codecs.pack_fp4(nib), sc)
    np.testing.assert_array_equal(y, wv[:, cols].T.astype(np.float32))


# ---------------------------------------------------------------------------
# structural identities on random data
# ---------------------------------------------------------------------------

def test_uniform_block_scales_make_blockwise_the_per_channel_recipe():
    """When every 128-block of a row has the row's absmax (so the per-block
    activation scales equal the per-token one) and the weight's block scales
    are its channel scale repeated, the blockwise result is the per-channel
    one up to float32 summation order: within one bf16 ulp."""
    from conftest import bf16_ulp

    rng = np.random.default_rng(16)
    m, k, n = 6, 1024, 40
    x = _bf(rng.standard_normal((m, k)).astype(np.float32))
    amax = np.abs(x).max(axis=1, keepdims=True)
    x[:, ::128] = amax  # every block reaches the row max
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    yc, xq_c, sx = linear.w8a8_per_channel(x, wq, ws, "fp8")
    yb, xq_b, xs = linear.w8a8_blockwise(x, wq, np.repeat(ws[:, None], k // 128, axis=1))
    np.testing.assert_array_equal(xq_c, xq_b)
    np.testing.assert_array_equal(np.repeat(sx[:, None], k // 128, axis=1), xs)
    assert (np.abs(yc - yb) <= bf16_ulp(np.maximum(np.abs(yc), np.abs(yb)))).all()
    # a per-channel scale applied along the wrong axis does not pass this
    yt, _, _ = linear.w8a8_per_channel(x, wq, np.roll(ws, 1), "fp8")
    assert not (np.abs(yc - yt) <= bf16_ulp(np.abs(yc))).all()


@pytest.mark.parametrize("fn", ["w8a8_fp8", "w8a8_int8", "w8a16", "w16a16"])
def test_output_columns_follow_weight_rows(fn):
    """Permuting the weight rows (with their scales) permutes the output
    columns and nothing else; the rows of x are independent of each other
    (a row's result does not change when the other rows change)."""
    rng = np.random.default_rng(17)
    m, k, n = 5, 256, 18
    x = _bf(rng.standard_normal((m, k)).astype(np.float32))
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    qd = "int8" if fn == "w8a8_int8" else "fp8"
    wq, ws = quant.quantize_tensor(w, qd)

    def run(xx, wwq, wws):
        if fn.startswith("w8a8"):
            return linear.w8a8_per_channel(xx, wwq, wws, qd)[0]
        if fn == "w8a16":
            return linear.w8a16_per_channel(xx, wwq, wws)
        return linear.w16a16(xx, _bf(quant.dequant_codes(wwq, qd) * wws[:, None]))

    y = run(x, wq, ws)
    perm = rng.permutation(n)
    np.testing.assert_array_equal(run(x, wq[perm], ws[perm]), y[:, perm])
    x2 = x.copy()
    x2[1:] *= 7.0
    np.testing.assert_array_equal(run(x2, wq, ws)[0], y[0])


def test_w4a4_mxfp4_known_answers_and_w4a16_identity():
    from oracle.quant import quantize_mx_fp4

    k, n = 128, 8
    # all ones (code 2, scale byte 127) on both sides: every output is K
    ones = np.full((3, k // 2), 0x22, np.uint8)
    s1 = np.full((3, k // 32), 127, np.uint8)
    wq = np.full((n, k // 2), 0x22, np.uint8)
    ws = np.full((n, k // 32), 127, np.uint8)
    np.testing.assert_array_equal(linear.w4a4_mxfp4(ones, s1, wq, ws), np.full((3, n), float(k), np.float32))
    # one-hot activation (1.0 at column c) reads back column c of the weight
    rng = np.random.default_rng(2)
    wq = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    ws = rng.integers(120, 130, (n, k // 32), dtype=np.uint8)
    wd = codecs.dequant_mxfp4(wq, ws)
    for c in (0, 1, 37, 127):
        x = np.zeros((1, k), np.float32)
        x[0, c] = 1.0
        aq, as_ = quantize_mx_fp4(x)
        np.testing.assert_array_equal(linear.w4a4_mxfp4(aq, as_, wq, ws)[0], codecs.bf16_round(wd[:, c]))
    # equal to the W4A16 recipe on the dequantized (bf16-exact) activations
    x = rng.standard_normal((5, k)).astype(np.float32)
    aq, as_ = quantize_mx_fp4(x)
    ad = codecs.dequant_mxfp4(aq, as_)
    assert np.array_equal(codecs.bf16_round(ad), ad)
    np.testing.assert_allclose(linear.w4a4_mxfp4(aq, as_, wq, ws), linear.w4a16_mxfp4(ad, wq, ws), rtol=2 ** -7,
                               atol=1e-6)
