"""Pins the oracle's codecs (CPU).

Known answers are the reference's own test vectors
(`tests/layers/core/test_mxfp4_requantization.py`); e4m3 / bf16 rounding is
pinned against torch's float8_e4m3fn / bfloat16 casts (library routines)
over dense sweeps that include every rounding boundary.
"""

import numpy as np
import pytest
import torch

from oracle import codecs


@pytest.mark.parametrize(
    "u8,expected",
    # test_mxfp4_requantization.py:194-209 values; 2**(b-127) in f32, 255 -> inf
    [(0, 2.0 ** -127), (1, 2.0 ** -126), (127, 1.0), (128, 2.0), (253, 2.0 ** 126),
     (254, 2.0 ** 127), (255, np.inf)],
)
def test_e8m0_known_values(u8, expected):
    got = codecs.e8m0_decode(np.array([u8], np.uint8))[0]
    assert got == np.float32(expected)


@pytest.mark.parametrize("byte_val", [0, 1, 15, 16, 128, 255])
def test_unpack_specific_bytes(byte_val):
    # test_mxfp4_requantization.py:230-239: low nibble first
    lut = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    got = codecs.fp4_decode(codecs.unpack_fp4(np.array([[byte_val]], np.uint8)))
    np.testing.assert_array_equal(got, [[lut[byte_val & 15], lut[byte_val >> 4]]])


def test_unpack_all_bytes_is_the_e2m1_format():
    # every code against the E2M1 definition: S.EE.M, bias 1, E=0 subnormal
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = (m * 0.5) if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert codecs.fp4_decode(np.array([c]))[0] == np.float32(-v if s else v)


@pytest.mark.parametrize("lo,hi", [(0, 0), (15, 15), (1, 0), (0, 1), (5, 10)])
def test_pack_specific_values(lo, hi):
    # test_mxfp4_requantization.py:371-387
    assert codecs.pack_fp4(np.array([[lo, hi]]))[0, 0] == (lo | (hi << 4))


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(42)
    idx = rng.integers(0, 16, (4, 64, 512))
    np.testing.assert_array_equal(codecs.unpack_fp4(codecs.pack_fp4(idx)), idx)


def test_dequant_mxfp4_blocks_scale_each_32():
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (8, 64), dtype=np.uint8)
    sc = rng.integers(100, 140, (8, 4), dtype=np.uint8)
    d = codecs.dequant_mxfp4(packed, sc)
    vals = codecs.fp4_decode(codecs.unpack_fp4(packed))
    for n in range(8):
        for k in range(128):
            assert d[n, k] == vals[n, k] * np.float32(2.0 ** (int(sc[n, k // 32]) - 127))


def _e4m3_sweep():
    # all codes' values, the midpoints between neighbours, and +-1 ulp around
    # each midpoint (the RNE tie and both sides), plus random values
    vals = codecs.e4m3_decode(np.arange(256, dtype=np.uint8))
    fin = np.unique(vals[np.isfinite(vals)].astype(np.float64))
    mids = (fin[:-1] + fin[1:]) / 2
    mids32 = mids.astype(np.float32)
    up = np.nextafter(mids32, np.float32(np.inf))
    dn = np.nextafter(mids32, np.float32(-np.inf))
    rnd = np.random.default_rng(0).uniform(-448, 448, 200000).astype(np.float32)
    tiny = np.random.default_rng(1).uniform(-2 ** -6, 2 ** -6, 50000).astype(np.float32)
    return np.concatenate([fin.astype(np.float32), mids32, up, dn, rnd, tiny,
                           np.float32([0.0, -0.0, 448.0, -448.0])])


def test_e4m3_encode_matches_torch_cast():
    x = _e4m3_sweep()
    x = x[np.abs(x) <= 448]
    ours = codecs.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, ref)


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(codecs.e4m3_decode(codes), ref)


def test_e4m3_known_values():
    assert codecs.e4m3_encode(np.float32([448.0]))[0] == 0x7E
    assert codecs.e4m3_encode(np.float32([2 ** -9]))[0] == 0x01
    assert codecs.e4m3_encode(np.float32([2 ** -6]))[0] == 0x08
    assert codecs.e4m3_encode(np.float32([np.nan]))[0] & 0x7F == 0x7F
    assert codecs.e4m3_encode(np.float32([-1.0]))[0] == 0xB8


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        # exact ties at bf16 granularity
                        (rng.integers(0, 2 ** 16, 5000).astype(np.uint32) << 16 | 0x8000).view(np.float32)])
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(codecs.bf16_round(x), ref)


# ---------------------------------------------------------------- NVFP4


def test_nvfp4_fused_scale_known_answers():
    """`tests/layers/adapter/quantization/test_nvfp4.py:255-284`: unit block
    scales times a 2.5 global give 2.5; MoE w13 takes the gate global on the
    first half of the rows and the up global on the second
    (`nvfp4.py:398-409`), w2 its per-expert global."""
    ones = np.ones((32, 4), np.float32)
    np.testing.assert_array_equal(codecs.nvfp4_fuse_scales(ones, np.float32(2.5)), ones * 2.5)
    s13 = codecs.nvfp4_fuse_scales(np.ones((2, 32, 4), np.float32), np.array([[2, 3], [4, 5]], np.float32),
                                   halves=True)
    np.testing.assert_array_equal(s13[:, :16], np.array([2, 4], np.float32)[:, None, None] * np.ones((2, 16, 4)))
    np.testing.assert_array_equal(s13[:, 16:], np.array([3, 5], np.float32)[:, None, None] * np.ones((2, 16, 4)))
    s2 = codecs.nvfp4_fuse_scales(np.ones((2, 8, 2), np.float32), np.array([2, 4], np.float32))
    np.testing.assert_array_equal(s2, np.array([2, 4], np.float32)[:, None, None] * np.ones((2, 8, 2)))
    # e4m3 codes decode first: 0x38 = 1.0, 0x3c = 1.5, 0x30 = 0.5
    codes = np.array([[0x38, 0x3C, 0x30, 0xB8]], np.uint8)
    np.testing.assert_array_equal(codecs.nvfp4_fuse_scales(codes, np.float32(2.0)),
                                  np.array([[2.0, 3.0, 1.0, -2.0]], np.float32))


def test_nvfp4_dequant_rounds_scale_then_product_to_bf16():
    """Block 16 is dequantized in bf16 (`kernels/megablox/gmm_v2.py:452-462`):
    bf16(code * bf16(scale)). Hand-computed cases: 1.5 x 1.0078125 =
    1.51171875 sits halfway between bf16 neighbours 1.5078125 and 1.515625
    and rounds to the even one (1.515625); 1.5 x 1.0234375 = 1.53515625 ties
    down to 1.53125; scale 1.005859375 rounds up to 1.0078125 first (without
    that step the product would round to 1.5078125)."""
    def one(code, scale):
        packed = np.array([[code | (code << 4)] * 8], np.uint8)  # one row, K = 16
        return codecs.dequant_nvfp4(packed, np.array([[scale]], np.float32))[0, 0]

    assert one(3, 1.0078125) == np.float32(1.515625)     # e2m1 code 3 = 1.5
    assert one(3, 1.0234375) == np.float32(1.53125)
    assert one(3, 1.005859375) == np.float32(1.515625)
    assert one(11, 1.0078125) == np.float32(-1.515625)  # code 11 = -1.5
    assert one(2, 1.005859375) == np.float32(1.0078125)  # code 2 = 1.0: just the rounded scale
    assert one(7, 3.0) == np.float32(18.0)               # code 7 = 6.0, exact


def test_nvfp4_dequant_with_power_of_two_scales_is_the_mxfp4_dequant():
    """With power-of-two scales every product is exact, so NVFP4 and MXFP4
    dequantization (pinned by the reference's e8m0 / e2m1 known answers)
    agree; the 16-wide blocks each take their own scale."""
    rng = np.random.default_rng(4)
    packed = rng.integers(0, 256, (8, 32), dtype=np.uint8)  # K = 64
    e = rng.integers(120, 134, (8, 2)).astype(np.uint8)     # e8m0 per 32 k
    mx = codecs.dequant_mxfp4(packed, e)
    s16 = np.repeat(codecs.e8m0_decode(e), 2, axis=1)       # the same scale on both 16-k halves
    np.testing.assert_array_equal(codecs.dequant_nvfp4(packed, s16), mx)
    s16[:, 1] *= 2  # second 16-k block of each row doubles
    nv = codecs.dequant_nvfp4(packed, s16)
    np.testing.assert_array_equal(nv[:, 16:32], mx[:, 16:32] * 2)
    np.testing.assert_array_equal(nv[:, :16], mx[:, :16])


# ---------------------------------------------------------------- INT4


def test_int4_packing_is_the_reference_tests_encoding():
    """`tests/kernels/test_gmm_v2.py:445-455`: nibble = (v + 8) & 15 at bits
    4i of carrier j for value 8j + i; XOR 0x88888888 turns the carriers into
    two's complement nibbles (what the reference's load hands to jnp.int4)."""
    vals = np.array([[-8, -1, 0, 1, 7, 3, -5, 2, 6, -7, 5, -2, 4, -3, -4, -6]], np.int64)
    c = codecs.int4_pack(vals)
    assert c.dtype == np.int32 and c.shape == (1, 2)
    # carrier 0: nibbles 0, 7, 8, 9, 15, 11, 3, 10 (low first)
    assert int(c[0, 0]) & 0xFFFFFFFF == 0xA3BF9870
    np.testing.assert_array_equal(codecs.int4_unpack(c), vals.astype(np.float32))
    np.testing.assert_array_equal(codecs.int4_unpack(c.view(np.uint8)), vals.astype(np.float32))
    x = (c.view(np.uint32) ^ np.uint32(0x88888888))
    nib = np.stack([(x >> (4 * i)) & 0xF for i in range(8)], axis=-1).reshape(1, 16).astype(np.int64)
    np.testing.assert_array_equal(np.where(nib >= 8, nib - 16, nib), vals)


def test_int4_dequant_rounds_the_bf16_product():
    """int4.astype(bf16) * bf16 scale (`tests/kernels/test_gmm_v2.py:434`):
    7 x 1.0078125 = 7.0546875 rounds up to 7.0625; -3 x 1.0078125 =
    -3.0234375 is a tie that goes to the even neighbour -3.03125; a scale that
    is not bf16 rounds first (1.005859375 -> 1.0078125)."""
    def one(v, scale):
        c = codecs.int4_pack(np.array([[v] * 32], np.int64))
        return codecs.dequant_int4(c, np.array([[scale]], np.float32))[0, 0]

    assert one(7, 1.0078125) == np.float32(7.0625)
    assert one(-3, 1.0078125) == np.float32(-3.03125)
    assert one(1, 1.005859375) == np.float32(1.0078125)
    assert one(-8, 0.5) == np.float32(-4.0)
    assert one(0, 3.0) == np.float32(0.0)


def test_e5m2_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy()
    got = codecs.e5m2_decode(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok], ref[ok])
    assert (np.signbit(got[ok]) == np.signbit(ref[ok])).all()


def test_e5m2_encode_matches_torch_cast():
    """RNE over random magnitudes across the whole range, the subnormals,
    every halfway point between adjacent codes, the overflow edge (61440
    rounds to inf), signed zeros, inf and NaN: the codes torch's
    float8_e5m2 cast gives."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(100000) * np.exp2(rng.integers(-20, 17, 100000))).astype(np.float32)
    vals = codecs.e5m2_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    fin = np.sort(vals[np.isfinite(vals) & (vals >= 0)])
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    edge = np.float32([57344.0, 61439.996, 61440.0, 65536.0, 2.0 ** -17, 3 * 2.0 ** -18, 0.0, -0.0,
                       np.inf, -np.inf, np.nan, -np.nan])
    x = np.concatenate([x, mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)), edge])
    ref = torch.from_numpy(x).to(torch.float8_e5m2).view(torch.uint8).numpy()
    np.testing.assert_array_equal(codecs.e5m2_encode(x), ref)
