"""Quantizers of the reference, restated in numpy.

Two different quantizers exist in the reference and they round differently:

* runtime activation quantization, `kernels/quantized_matmul/util.py:294-318`
  (`quantize_block`): ``scale = absmax / qmax`` (a DIVISION), codes
  ``x / scale``. JAX type promotion decides the arithmetic precision: for a
  float target, ``get_max_min`` returns a NumPy float32 scalar, which is not
  weakly typed, so a bf16 ``x`` is promoted and everything runs in float32;
  for an int8 target it returns a Python int, which IS weakly typed, so the
  whole computation stays in bf16 (every intermediate rounded to bf16).
* load-time weight quantization, `layers/core/quantization.py:232-318`
  (`quantize_tensor`): ``scale = absmax * f32(1/qmax)`` (a RECIPROCAL
  MULTIPLY), ``inv = where(scale == 0, 0, 1/scale)``, codes
  ``clamp(x * inv)``; integer targets round half-to-even first.

Test infrastructure only.
"""

import numpy as np

from oracle.codecs import bf16_round, e4m3_decode, e4m3_encode, e5m2_decode, e5m2_encode

FP8_MAX = np.float32(448.0)
E5M2_MAX = np.float32(57344.0)


def _absmax(x, axis):
    return np.max(np.abs(x), axis=axis, keepdims=True)


def quantize_block_fp8(x, axis=-1):
    """`util.py:303-318` with a float8_e4m3fn target (float32 arithmetic).

    ``x`` holds bf16 values as float32. Returns (uint8 e4m3 codes, f32 scale
    with the reduced axis kept).
    """
    x = np.asarray(x, dtype=np.float32)
    scale = (_absmax(x, axis) / FP8_MAX).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = np.clip((x / scale).astype(np.float32), -FP8_MAX, FP8_MAX)
    return e4m3_encode(q), scale


def quantize_block_int8(x, axis=-1):
    """`util.py:303-318` with an int8 target (bf16 arithmetic).

    Every intermediate is rounded to bf16 because ``qmax`` (127) is a weakly
    typed Python int: ``scale = bf16(absmax / 127)``, ``q = round_half_even(
    bf16(x / scale))``. A float32 division followed by one bf16 rounding equals
    the correctly rounded bf16 quotient (24 >= 2*8+2 bits, so the double
    rounding is innocuous). Returns (int8 codes, f32 scale = f32(bf16 scale)).

    parity unpinned: the bf16 quotient can reach 127.5, which rounds to 128;
    the reference then casts with XLA's float->int8 convert, assumed
    saturating here (128 -> 127).
    """
    x = bf16_round(np.asarray(x, dtype=np.float32))
    scale = bf16_round(_absmax(x, axis) / np.float32(127.0))
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    with np.errstate(invalid="ignore"):
        q = np.rint(bf16_round(x / scale))
    q = np.where(np.isnan(q), 0, np.clip(q, -128, 127)).astype(np.int8)  # NaN -> 0
    return q, scale


def quantize_block_e5m2(x, axis=-1):
    """`util.py:303-318` with a float8_e5m2 target: as the e4m3 form (the
    finfo maximum is a NumPy float32 scalar, so float32 arithmetic) with
    qmax = 57344, the e5m2 maximum."""
    x = np.asarray(x, dtype=np.float32)
    scale = (_absmax(x, axis) / E5M2_MAX).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = np.clip((x / scale).astype(np.float32), -E5M2_MAX, E5M2_MAX)
    return e5m2_encode(q), scale


def quantize_act(x, qdtype, block=None):
    """Per-token (``block=None``) or per-(token, block) activation quant.

    ``qdtype`` is "fp8", "e5m2" or "int8". Returns codes [M, K] and scales
    [M] or [M, K/block] (float32).
    """
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    fn = {"fp8": quantize_block_fp8, "e5m2": quantize_block_e5m2, "int8": quantize_block_int8}[qdtype]
    if block is None:
        q, s = fn(x, axis=-1)
        return q, s[:, 0]
    q, s = fn(x.reshape(m, k // block, block), axis=-1)
    return q.reshape(m, k), s[..., 0]


GMM_LHS_BLOCK = 512


def quantize_gmm_lhs(x, qdtype, block=GMM_LHS_BLOCK):
    """The grouped matmul's on-the-fly activation quant,
    `kernels/megablox/gmm_v2.py:508-536` (taken when the weight's quant
    block is 256 columns or more, per-channel included, `:1198-1218`;
    `quant_block_size=512`, `:1222-1228`).

    Per (row, 512-column block) from column 0 (the kernel's K tile is the
    whole K, `:966-969`, so the last block is partial when K % 512 != 0),
    in the activation's dtype, bf16 (``dtype_max`` is a Python float, so the
    division stays bf16): ``scale = bf16(absmax / qmax)``; ``inv = 0`` where
    the scale is 0 else ``bf16(1 / scale)``; ``q = (x * inv).astype(q)``:
    e4m3 round-to-nearest-even of the bf16 product (no clip; |q| <= ~452 <
    464, the e4m3 overflow threshold), int8 by truncation toward zero (the
    float -> int cast). A f32 quotient rounded once to bf16 is the correctly
    rounded bf16 quotient (24 >= 2*8 + 2 bits).

    Returns (codes [M, K] uint8 e4m3 / int8, scales f32 [M, ceil(K/512)]
    holding the bf16 values; a zero block keeps scale 0).
    """
    x = bf16_round(np.asarray(x, dtype=np.float32))
    m, k = x.shape
    nb = (k + block - 1) // block
    qmax = np.float32(448.0 if qdtype == "fp8" else 127.0)
    codes = np.zeros((m, k), np.uint8 if qdtype == "fp8" else np.int8)
    scales = np.zeros((m, nb), np.float32)
    for b in range(nb):
        xb = x[:, b * block:(b + 1) * block]
        amax = np.max(np.abs(xb), axis=1, keepdims=True)
        scale = bf16_round((amax / qmax).astype(np.float32))
        with np.errstate(divide="ignore"):
            inv = np.where(scale == 0, np.float32(0.0), bf16_round((np.float32(1.0) / scale).astype(np.float32)))
        v = bf16_round((xb * inv).astype(np.float32))
        if qdtype == "fp8":
            codes[:, b * block:(b + 1) * block] = e4m3_encode(v)
        else:
            t = np.where(np.isnan(v), 0, np.clip(np.trunc(v), -128, 127))
            codes[:, b * block:(b + 1) * block] = t.astype(np.int8)
        scales[:, b] = scale[:, 0]
    return codes, scales


def dequant_codes(q, qdtype) -> np.ndarray:
    if qdtype == "fp8":
        return e4m3_decode(q)
    if qdtype == "e5m2":
        return e5m2_decode(q)
    return np.asarray(q, dtype=np.int8).astype(np.float32)


def quantize_tensor(w, qdtype, block=None):
    """Load-time quantizer, `layers/core/quantization.py:232-318` (no ue8m0).

    ``qdtype``: "fp8" (e4m3fn), "e5m2" or "int8" (qmax the dtype's finfo /
    iinfo maximum). Quantizes along the last axis; ``block=None`` means the whole axis.
    Returns (codes, scale) with scale shaped [..., K/block] (squeezed to [...]
    for the whole-axis case, as the reference's ``squeeze(-1)`` does).
    """
    w = np.asarray(w, dtype=np.float32)
    k = w.shape[-1]
    block = block or k
    if k % block:
        raise ValueError("Quantization expects the requested axis to be divisible by block_size")
    qmax = {"fp8": 448.0, "e5m2": 57344.0, "int8": 127.0}[qdtype]
    qmin = -128.0 if qdtype == "int8" else -qmax
    blocked = w.reshape(*w.shape[:-1], k // block, block)
    recip = np.float32(1.0 / qmax)
    scale = (_absmax(blocked, -1) * recip).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(scale == 0, np.float32(0.0), (np.float32(1.0) / scale)).astype(np.float32)
    q = np.clip((blocked * inv).astype(np.float32), qmin, qmax)
    if qdtype == "fp8":
        codes = e4m3_encode(q)
    elif qdtype == "e5m2":
        codes = e5m2_encode(q)
    else:
        codes = np.where(np.isnan(q), 0, np.rint(q)).astype(np.int8)
    codes = codes.reshape(w.shape)
    scale = scale[..., 0]
    if block == k:
        scale = scale[..., 0]
    return codes, scale


def quantize_fp8_tiles(w, tile=128):
    """DeepSeek-V3 checkpoint form of a weight: one f32 scale per 128x128 tile.

    ``scale_inv = amax(tile) / 448`` (the checkpoint's ``weight_scale_inv``),
    codes = RNE e4m3 of ``w / scale_inv`` clipped to +-448. This generates the
    BASELINE config-2/4 inputs; it is not a reference function.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    t = w.reshape(n // tile, tile, k // tile, tile)
    s = (np.max(np.abs(t), axis=(1, 3)) / FP8_MAX).astype(np.float32)
    s = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    q = np.clip(t / s[:, None, :, None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3_encode(q).reshape(n, k), s


def dequant_tiles(codes, scale_inv, tile=128) -> np.ndarray:
    """f32 weights from e4m3 codes [N, K] and tile scales [N/tile, K/tile].

    `adapter/quantization/fp8.py:132-182` (`_dequantize_fp8_linear`, block
    branch): code value times the scale of its tile.
    """
    n, k = codes.shape
    v = e4m3_decode(codes).reshape(n // tile, tile, k // tile, tile)
    return (v * scale_inv[:, None, :, None]).reshape(n, k).astype(np.float32)


# ---------------------------------------------------------------- MX (e2m1 + e8m0) activations

MX_BLOCK = 32
FP4_MAX = np.float32(6.0)
# bucket edges of the reference's e2m1 encoder: magnitude code = number of
# edges strictly below |v| (torch.bucketize, right=False), so a value on an
# edge takes the lower code
FP4_EDGES = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)


def e8m0_exponent_ceil(scale) -> np.ndarray:
    """Smallest e in [-127, 127] with 2**e >= scale (f32 scale >= 0).

    `layers/core/quantization.py:285-298`: ``ceil(log2(scale))``, raised by
    one where ``exp2`` of it is still below the scale, clamped to [-127,
    127]; a zero scale gives -inf and the clamp pins it to -127. Computed
    here exactly from the binary exponent (frexp: scale = f * 2**E with f in
    [0.5, 1), so the answer is E - 1 when f == 0.5, else E), which is the
    value that rule repairs ``log2`` to.
    """
    s = np.asarray(scale, dtype=np.float32)
    f, e = np.frexp(s)
    out = np.where(f == 0.5, e - 1, e).astype(np.int64)
    out = np.where(s == 0, -127, out)
    out = np.where(np.isinf(s), 127, out)
    return np.clip(out, -127, 127)


def fp4_encode_bucket(v) -> np.ndarray:
    """Scaled f32 values -> e2m1 nibbles, the reference's encoder
    `compressed_tensors_moe/utils.py:167-183` (`quantize_to_fp4_e2m1_nibbles`):
    magnitude by the bucket edges above (values past 5.0, including those
    beyond 6, saturate to code 7 = 6.0), sign bit 8 for v < 0 (so -0.0
    keeps sign 0)."""
    v = np.asarray(v, dtype=np.float32)
    mag = np.searchsorted(FP4_EDGES, np.abs(v), side="left").astype(np.uint8)
    return (mag | np.where(v < 0, np.uint8(8), np.uint8(0))).astype(np.uint8)


def quantize_mx_fp4(x, k_pad=None):
    """bf16 / f32 activations [M, K] -> MXFP4 (packed e2m1 codes [M, Kp/2],
    low nibble = even k; e8m0 bytes [M, Kp/32]).

    The reference's ue8m0 block quantizer, `layers/core/quantization.py:
    232-318` (`quantize_tensor(..., block_size=32, use_ue8m0=True)`) with
    e2m1 as the target (qmax 6): per 32-value block ``scale = amax * f32(1/6)``
    in f32, snapped UP to a power of two 2**e (`e8m0_exponent_ceil`), byte
    e + 127; values ``x * (1 / 2**e)`` clamped to +-6 and encoded by the
    reference's e2m1 encoder (`fp4_encode_bucket`). The reference has no
    activation quantizer for its W4A4 method (it runs W4A16); this is its
    weight-side rule applied to activations. Columns K..Kp-1 (``k_pad``, a
    multiple of 32 >= K) are zero blocks: codes 0, byte 0 (the rule's answer
    for an all-zero block).

    A block holding an inf or NaN (the reference's rule has no answer: its
    scale would be non-finite) gets this build's definition: codes 0 and
    byte 255, the e8m0 NaN encoding, so the block dequantizes to NaN and the
    row's other blocks are untouched. Parity of that case is the build's own
    definition (no reference counterpart).
    """
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    kp = k if k_pad is None else int(k_pad)
    if k % MX_BLOCK or kp % MX_BLOCK or kp < k:
        raise ValueError("MX quantization needs K and the padded K to be multiples of 32")
    xp = np.zeros((m, kp), np.float32)
    xp[:, :k] = x
    blocks = xp.reshape(m, kp // MX_BLOCK, MX_BLOCK)
    bad = ~np.isfinite(blocks).all(axis=-1)
    blocks = np.where(bad[..., None], np.float32(0.0), blocks)
    amax = np.max(np.abs(blocks), axis=-1)
    scale = (amax * np.float32(1.0 / 6.0)).astype(np.float32)
    e = e8m0_exponent_ceil(scale)
    inv = np.ldexp(np.float32(1.0), -e).astype(np.float32)
    v = np.clip((blocks * inv[..., None]).astype(np.float32), -FP4_MAX, FP4_MAX)
    codes = fp4_encode_bucket(v).reshape(m, kp)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return packed, np.where(bad, 255, e + 127).astype(np.uint8)
