"""Bit-level codecs: bf16 rounding, OCP e4m3fn and e5m2, e2m1 (fp4), e8m0.

Written from the format definitions (OCP 8-bit floating point spec v1.0 for
E4M3 "fn" and E5M2; OCP MX spec v1.0 for E2M1 and E8M0). Test
infrastructure only.
"""

import numpy as np

# ---------------------------------------------------------------- bfloat16


def bf16_round(x) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), return f32.

    NaN stays NaN (quiet). This is the rounding every bf16 cast in the
    reference performs (torch `.to(bfloat16)`, jnp `.astype(bfloat16)`).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def bf16_bits(x) -> np.ndarray:
    """bf16 bit patterns (uint16) of float32 values after RNE rounding."""
    r = bf16_round(x)
    return (r.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


# ---------------------------------------------------------------- e4m3fn

E4M3_MAX = 448.0
E4M3_NAN = 0x7F


def _e4m3_values(c) -> np.ndarray:
    """Layout S.EEEE.MMM, bias 7, no infinities, S.1111.111 is NaN."""
    c = np.asarray(c, dtype=np.int64)
    s = np.where((c >> 7) & 1, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = s * val
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return val.astype(np.float32)


_E4M3_TABLE = _e4m3_values(np.arange(256))


def e4m3_decode(codes) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (exact), through the table of
    `_e4m3_values` over all 256 codes."""
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x) -> np.ndarray:
    """float32 -> uint8 e4m3fn codes, round-to-nearest-even.

    Magnitudes that round above 448 and NaN inputs encode as NaN (0x7F/0xFF),
    as torch's float8_e4m3fn cast does; every caller in the reference clips to
    +-448 first, so only NaN reaches that branch on the hot path.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.int64) << 7
    _, ex = np.frexp(a)  # a = f * 2**ex, f in [0.5, 1)
    e = ex.astype(np.int64) - 1  # a in [2**e, 2**(e+1))
    e = np.maximum(e, -6)  # subnormal binade shares the 2**-9 quantum
    q = np.exp2((e - 3).astype(np.float64))
    r = np.rint(a / q)  # exact quotient (a is f32, q a power of 2); RNE
    v = r * q  # the rounded magnitude, exactly representable
    code = np.zeros(a.shape, dtype=np.int64)
    nz = v > 0
    _, ev = np.frexp(np.where(nz, v, 1.0))
    ev = ev.astype(np.int64) - 1
    sub = nz & (ev < -6)
    code = np.where(sub, np.rint(v / 2.0 ** -9).astype(np.int64), code)
    norm = nz & ~sub
    mant = np.rint(v / np.exp2((ev - 3).astype(np.float64))).astype(np.int64) - 8
    code = np.where(norm, ((ev + 7) << 3) | mant, code)
    code = np.where(np.isnan(x) | (v > E4M3_MAX), E4M3_NAN, code)
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------- e5m2

E5M2_MAX = 57344.0
E5M2_INF = 0x7C
E5M2_NAN = 0x7F


def _e5m2_values(c) -> np.ndarray:
    """Layout S.EEEEE.MM, bias 15, IEEE-like: E == 31 is inf (M == 0) or NaN."""
    c = np.asarray(c, dtype=np.int64)
    s = np.where((c >> 7) & 1, -1.0, 1.0)
    e = (c >> 2) & 0x1F
    m = c & 0x3
    with np.errstate(over="ignore"):
        val = np.where(e == 0, m * 2.0 ** -16, (1.0 + m / 4.0) * np.exp2(e - 15.0))
    val = np.where(e == 0x1F, np.where(m == 0, np.inf, np.nan), val)
    return (s * val).astype(np.float32)


_E5M2_TABLE = _e5m2_values(np.arange(256))


def e5m2_decode(codes) -> np.ndarray:
    """uint8 e5m2 codes -> float32 values (exact)."""
    return _E5M2_TABLE[np.asarray(codes, dtype=np.uint8)]


def e5m2_encode(x) -> np.ndarray:
    """float32 -> uint8 e5m2 codes, round-to-nearest-even; magnitudes that
    round above 57344 become inf, NaN becomes 0x7F with its sign (torch's
    float8_e5m2 cast). The reference clips to +-57344 first."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.int64) << 7
    _, ex = np.frexp(a)
    e = np.maximum(ex.astype(np.int64) - 1, -14)  # subnormal binade: quantum 2**-16
    q = np.exp2((e - 2).astype(np.float64))
    v = np.rint(a / q) * q  # RNE, exact
    code = np.zeros(a.shape, dtype=np.int64)
    nz = v > 0
    _, ev = np.frexp(np.where(nz, v, 1.0))
    ev = ev.astype(np.int64) - 1
    sub = nz & (ev < -14)
    code = np.where(sub, np.rint(v / 2.0 ** -16).astype(np.int64), code)
    norm = nz & ~sub
    mant = np.rint(v / np.exp2((ev - 2).astype(np.float64))).astype(np.int64) - 4
    code = np.where(norm, ((ev + 15) << 2) | mant, code)
    code = np.where(v > E5M2_MAX, E5M2_INF, code)
    code = np.where(np.isnan(x), E5M2_NAN, code)
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------- e2m1 / e8m0

# Value of each 4-bit e2m1 code: S.EE.M, bias 1; E==0 is subnormal (0, 0.5).
FP4_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


def fp4_decode(nibbles) -> np.ndarray:
    """4-bit codes -> float32 (`layers/core/quantization.py:145-175`)."""
    return FP4_VALUES[np.asarray(nibbles, dtype=np.int64) & 0xF]


def unpack_fp4(packed) -> np.ndarray:
    """uint8 [..., K/2] -> 4-bit codes [..., K], low nibble first.

    `layers/core/quantization.py:131-179` (`unpack_uint8_to_fp4`): element 2i
    is the low nibble of byte i, element 2i+1 the high nibble.
    """
    p = np.asarray(packed, dtype=np.uint8)
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    return np.stack([lo, hi], axis=-1).reshape(*p.shape[:-1], -1)


def pack_fp4(codes) -> np.ndarray:
    """4-bit codes [..., K] -> uint8 [..., K/2] (`quantization.py:445-468`)."""
    c = np.asarray(codes, dtype=np.uint8) & 0xF
    c = c.reshape(*c.shape[:-1], -1, 2)
    return (c[..., 0] | (c[..., 1] << 4)).astype(np.uint8)


def e8m0_decode(u8) -> np.ndarray:
    """e8m0 byte -> float32 2**(b-127) (`layers/core/quantization.py:105-128`).

    The reference computes `ldexp(1, b-127)` in float32, so b == 255 gives
    +inf (not NaN) and b == 0 gives the subnormal 2**-127.
    """
    b = np.asarray(u8, dtype=np.uint8).astype(np.int64)
    return np.ldexp(np.float32(1.0), b - 127).astype(np.float32)


def dequant_mxfp4(packed, scales_u8) -> np.ndarray:
    """MXFP4 [N, K/2] codes + e8m0 [N, K/32] -> float32 [N, K].

    `layers/core/quantization.py:321-345` (`dequantize_mxfp4_packed`): LUT
    value times the block's power of two; every product is exact in f32.
    """
    vals = fp4_decode(unpack_fp4(packed))
    s = e8m0_decode(scales_u8)
    n, k = vals.shape[-2], vals.shape[-1]
    blk = k // s.shape[-1]
    out = vals.reshape(*vals.shape[:-1], s.shape[-1], blk) * s[..., None]
    return out.reshape(*vals.shape[:-2], n, k).astype(np.float32)


# ---------------------------------------------------------------- NVFP4


def nvfp4_fuse_scales(block_scale, global_scale, halves=False):
    """ModelOpt NVFP4 block scales -> float32 fused scales.

    ``block_scale``: e4m3fn codes (uint8) or their float32 values, [..., N, K/16];
    ``global_scale``: the per-tensor float32 ``weight_scale_2`` -- a scalar for a
    linear (`layers/adapter/quantization/nvfp4.py:700-714`), [E] for MoE w2, or
    [E, 2] for MoE w13 with ``halves`` (gate rows take column 0, up rows column
    1, `nvfp4.py:398-409`). One float32 product per scale.
    """
    b = np.asarray(block_scale)
    b = e4m3_decode(b) if b.dtype == np.uint8 else b.astype(np.float32)
    g = np.asarray(global_scale, np.float32)
    if halves:
        n = b.shape[-2] // 2
        gate = (b[..., :n, :] * g[..., 0, None, None]).astype(np.float32)
        up = (b[..., n:, :] * g[..., 1, None, None]).astype(np.float32)
        return np.concatenate([gate, up], axis=-2)
    if g.ndim == 0:
        return (b * g).astype(np.float32)
    return (b * g.reshape(g.shape + (1,) * (b.ndim - g.ndim))).astype(np.float32)


def dequant_nvfp4(packed, scales_f32) -> np.ndarray:
    """NVFP4 [..., N, K/2] codes + float32 [..., N, K/16] scales -> the bf16
    weights (as float32) the reference multiplies with.

    Block 16 is below the MXU width, so `kernels/megablox/gmm_v2.py:452-462`
    dequantizes in the activation dtype: the scale is cast to bf16, the codes
    to bf16 (exact), and their bf16 product is rounded once to bf16.
    """
    vals = fp4_decode(unpack_fp4(packed))
    s = bf16_round(np.asarray(scales_f32, np.float32))
    n, k = vals.shape[-2], vals.shape[-1]
    blk = k // s.shape[-1]
    prod = vals.reshape(*vals.shape[:-1], s.shape[-1], blk) * s[..., None]
    return bf16_round(prod.reshape(*vals.shape[:-2], n, k).astype(np.float32))


# ---------------------------------------------------------------- INT4 (compressed-tensors)


def int4_pack(values) -> np.ndarray:
    """Symmetric int4 values [..., K] (-8..7) -> int32 carriers [..., K/8] in
    the compressed-tensors encoding the reference's test builds
    (`tests/kernels/test_gmm_v2.py:445-452`): nibble = (v + 8) & 15, value
    8j + i of a row in bits 4i..4i+3 of carrier j."""
    v = np.asarray(values, np.int64)
    u = (v + 8) & 0xF
    u = u.reshape(*u.shape[:-1], u.shape[-1] // 8, 8)
    words = np.sum(u << (4 * np.arange(8, dtype=np.int64)), axis=-1)
    return words.astype(np.uint32).view(np.int32)


def int4_unpack(carriers) -> np.ndarray:
    """int32 carriers [..., K/8] (or their bytes, uint8 [..., K/2]) -> int4
    values [..., K] as float32 (nibble - 8)."""
    c = np.ascontiguousarray(carriers)
    b = c.view(np.uint8) if c.dtype != np.uint8 else c  # little-endian: carrier j = bytes 4j..4j+3
    lo, hi = b & 0xF, b >> 4
    nib = np.stack([lo, hi], axis=-1).reshape(*b.shape[:-1], b.shape[-1] * 2)
    return nib.astype(np.float32) - 8.0


def dequant_int4(carriers, scales) -> np.ndarray:
    """INT4 weights + bf16-valued scales [..., N, K/group] -> the bf16 weights
    (as float32) the reference multiplies with: groups below 256 k are
    dequantized in the bf16 activation dtype, `int4.astype(bf16) * scale`
    (`kernels/megablox/gmm_v2.py:452-462`, the expected value of
    `tests/kernels/test_gmm_v2.py:434`), one bf16 rounding of the product."""
    vals = int4_unpack(carriers)
    s = bf16_round(np.asarray(scales, np.float32))
    n, k = vals.shape[-2], vals.shape[-1]
    grp = k // s.shape[-1]
    prod = vals.reshape(*vals.shape[:-1], s.shape[-1], grp) * s[..., None]
    return bf16_round(prod.reshape(*vals.shape[:-2], n, k).astype(np.float32))
