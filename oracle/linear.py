"""Dense quantized linear references (dequantize-then-matmul, fp32).

Weights are held N-major ``[N, K]`` here (the checkpoint layout); the
reference's runtime contraction over its K-major ``[K, N]`` copy computes the
same sums. Test infrastructure only.
"""

import numpy as np

from oracle.codecs import bf16_round, dequant_int4, dequant_mxfp4, dequant_nvfp4, e4m3_decode
from oracle.quant import GMM_LHS_BLOCK, dequant_codes, quantize_act, quantize_gmm_lhs


def _mm(a, b_nk) -> np.ndarray:
    """float32 [M, K] @ [N, K]^T with float32 accumulation (BLAS sgemm)."""
    return np.matmul(np.asarray(a, np.float32), np.asarray(b_nk, np.float32).T)


def w8a8_per_channel(x, wq, ws, qdtype):
    """`kernels/quantized_matmul/util.py:80-124` (`xla_quantized_matmul`).

    ``xq, sx = quantize_tensor(x)`` per token; ``dot(xq, wq)`` accumulated in
    int32 (int8) or float32 (fp8); ``.astype(f32) * sx``; ``* ws[None, :]``;
    cast to bf16. For int8 the integer dot is exact (computed in float64,
    exact below 2**53), so the float32 epilogue, done in the reference's
    operation order, reproduces the reference's output bit for bit.

    Returns (y as bf16-valued f32 [M, N], xq, sx).
    """
    xq, sx = quantize_act(x, qdtype)
    if qdtype == "int8":
        acc = np.matmul(xq.astype(np.float64), np.asarray(wq, np.int8).astype(np.float64).T)
        out = acc.astype(np.float32)
    else:  # e4m3 or e5m2 on both operands (the activation takes the weight's dtype)
        out = _mm(dequant_codes(xq, qdtype), dequant_codes(wq, qdtype))
    out = (out * sx[:, None]).astype(np.float32)
    out = (out * np.asarray(ws, np.float32)[None, :]).astype(np.float32)
    return bf16_round(out), xq, sx


def w8a16_per_channel(x, wq, ws, qdtype="fp8"):
    """`util.py:116-124` (``quantize_activation=False``): bf16 x times the
    weight codes, f32 accumulation, ``* ws``, bf16 out."""
    out = _mm(x, dequant_codes(wq, qdtype))
    out = (out * np.asarray(ws, np.float32)[None, :]).astype(np.float32)
    return bf16_round(out)


def w8a8_blockwise(x, wq, ws_blocks, block=128, round_out=True):
    """`tests/kernels/test_quantized_matmul_kernel.py:66-94`
    (`reference_block_quantized_matmul`), the oracle of the blockwise kernel
    `kernels/quantized_matmul/blockwise_kernel.py:197-247`.

    x is quantized per (token, block) to e4m3 in float32 (`util.quantize_block`
    on ``x.reshape(M, K/B, B)``); for each K block the f32 dot of codes is
    multiplied by ``x_s`` and ``w_s`` and the blocks are summed.

    ``ws_blocks`` is the per-(n, K-block) scale ``[N, K/B]`` (a 128x128 tile
    scale repeated along N is the DeepSeek-V3 case). Returns (y, xq, xs); y is
    the bf16-rounded output, or the float32 sums with ``round_out=False`` (the
    input of a fused activation).
    """
    m, k = x.shape
    n = wq.shape[0]
    xq, xs = quantize_act(x, "fp8", block=block)
    xv = e4m3_decode(xq).reshape(m, k // block, block)
    wv = e4m3_decode(wq).reshape(n, k // block, block)
    out = np.zeros((m, n), np.float32)
    for b in range(k // block):
        d = _mm(xv[:, b, :], wv[:, b, :])
        out += (d * xs[:, b:b + 1]).astype(np.float32) * ws_blocks[None, :, b]
    return (bf16_round(out) if round_out else out), xq, xs


def tile_scales_to_blocks(scale_tiles, n, tile=128):
    """[N/128, K/128] tile scales -> per-(n, K-block) [N, K/128]."""
    return np.repeat(np.asarray(scale_tiles, np.float32), tile, axis=0)[:n]


def w4a16_mxfp4(x, packed, scales_u8, bias=None):
    """MXFP4 weight x bf16 activation (`adapter/linear_common.py:188-209` ->
    `kernels/megablox/gmm_v2.py:452-462`: block 32 < MXU width, so the rhs is
    dequantized (exactly) in the activation dtype and bf16 x stays unquantized,
    f32 accumulation, bf16 out)."""
    w = dequant_mxfp4(packed, scales_u8)
    out = _mm(x, w)
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)


def w4a16_nvfp4(x, packed, scales_f32, bias=None):
    """NVFP4 weight x bf16 activation (`adapter/quantization/nvfp4.py:752-761`
    -> `quantized_matmul_fp4` -> gmm_v2 with block 16: the rhs is dequantized
    to bf16 as ``dequant_nvfp4`` states, bf16 x, f32 accumulation, bf16 out)."""
    out = _mm(x, dequant_nvfp4(packed, scales_f32))
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)


def w4a16_int4(x, carriers, scales, bias=None):
    """Packed-int4 weight x bf16 activation (gmm_v2 with ``rhs_quant_dtype``
    int4 and a group below 256: ``dequant_int4`` weights, bf16 x, f32
    accumulation, bf16 out)."""
    out = _mm(x, dequant_int4(carriers, scales))
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)


def w16a16(x, w, bias=None):
    """Unquantized bf16 linear with f32 accumulation."""
    out = _mm(x, w)
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)


def _block_dots(xq, wq, qdtype, block, wdtype=None):
    """Per-512-block dot products of codes: [blocks, M, N] float64 (exact:
    int8 products summed in float64 are exact integers, e4m3 / e5m2
    products have at most 8-bit significands)."""
    xv = dequant_codes(xq, qdtype).astype(np.float64)
    wv = dequant_codes(wq, wdtype or qdtype).astype(np.float64)
    k = xv.shape[1]
    nb = (k + block - 1) // block
    return np.stack([xv[:, b * block:(b + 1) * block] @ wv[:, b * block:(b + 1) * block].T for b in range(nb)])


def w8a8_gmm(x, wq, ws, qdtype, bias=None, round_out=True, wdtype=None):
    """The grouped matmul's quantized-lhs regime with per-channel weights
    (``ws`` [N]) or per-(row, B columns) weights (``ws`` [N, K/B], B a
    multiple of 512; `kernels/megablox/gmm_v2.py:500-548`), accumulated in
    float32: the
    activation codes and scales of `quantize_gmm_lhs`, each 512-column block's
    dot times its activation scale, summed over blocks, times the per-channel
    weight scale. This is the fp32-accumulated form the kernel computes (same
    codes, so only the summation differs); `w8a8_gmm_bf16acc` is the
    reference's own bf16 accumulation.

    ``qdtype`` is the activation codes' dtype ("fp8" for any float weight,
    e5m2 included: `gmm_v2.py:1198-1218`; "int8" for int8 weights) and
    ``wdtype`` the weight codes' (default the same).

    Returns (y [M, N] bf16-valued f32, or f32 sums with round_out=False; xq; xs).
    """
    xq, xs = quantize_gmm_lhs(x, qdtype)
    dots = _block_dots(xq, wq, qdtype, GMM_LHS_BLOCK, wdtype)
    ws = np.asarray(ws, np.float32)
    acc = np.zeros(dots.shape[1:], np.float32)
    if ws.ndim == 2:  # per (row, B columns): each 512-column block meets the weight block it lies in
        bw = xq.shape[1] // ws.shape[1]
        for b in range(dots.shape[0]):
            acc += ((dots[b].astype(np.float32) * xs[:, b:b + 1]).astype(np.float32)
                    * ws[None, :, b * GMM_LHS_BLOCK // bw])
        out = acc
    else:
        for b in range(dots.shape[0]):
            acc += (dots[b].astype(np.float32) * xs[:, b:b + 1]).astype(np.float32)
        out = (acc * ws[None, :]).astype(np.float32)
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return (bf16_round(out) if round_out else out), xq, xs


def w8a8_gmm_bf16acc(x, wq, ws, qdtype, bias=None):
    """`kernels/megablox/gmm_v2.py:508-560` as written: the accumulator is
    bf16 (`acc_dtype` defaults to bf16 when the lhs is quantized,
    `:1230-1237`): per 512-column block, ``bf16(dot)``, times the bf16
    activation scale (rounded), times the weight scale cast to bf16
    (rounded), added to the bf16 accumulator (rounded); the bias is added in
    bf16. Parity tests hold the kernel's fp32 accumulation to this within the
    north-star bar."""
    xq, xs = quantize_gmm_lhs(x, qdtype)
    dots = _block_dots(xq, wq, qdtype, GMM_LHS_BLOCK)
    ws16 = bf16_round(np.asarray(ws, np.float32))[None, :]
    acc = np.zeros(dots.shape[1:], np.float32)
    for b in range(dots.shape[0]):
        blk = bf16_round(dots[b].astype(np.float32))
        blk = bf16_round(blk * xs[:, b:b + 1])
        blk = bf16_round(blk * ws16)
        acc = bf16_round(acc + blk)
    if bias is not None:
        acc = bf16_round(acc + bf16_round(np.asarray(bias, np.float32))[None, :])
    return acc


def w8a16_blockwise(x, wq, ws_blocks, block=128, bias=None):
    """The grouped matmul's dequantize-before-matmul regime for FP8 weights
    with quant blocks under 256 columns (`kernels/megablox/gmm_v2.py:452-462`;
    the single-group call of `adapter/linear_common.py:88-114` with
    ``REQUANTIZE_BLOCK_SIZE=128``): each weight is ``bf16(code *
    bf16(scale))`` (the codes and scales cast to the bf16 activation dtype,
    multiplied in bf16), bf16 activations unquantized, f32 accumulation,
    bf16 out. ``ws_blocks`` is [N, K/block]."""
    w = dequant_codes(wq, "fp8")
    n, k = w.shape
    s = np.repeat(bf16_round(np.asarray(ws_blocks, np.float32)), block, axis=1)[:, :k]
    out = _mm(x, bf16_round((w * s).astype(np.float32)))
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)


def w4a4_mxfp4(a_packed, a_scales, w_packed, w_scales, bias=None):
    """MXFP4 activation x MXFP4 weight (the opt-in W4A4 regime): both
    operands dequantized exactly (`dequant_mxfp4`, `layers/core/
    quantization.py:321-345`), f64 sums of the exact products, bias in f32,
    bf16 out. Equal to `w4a16_mxfp4` of the dequantized activations (they
    are exact in bf16) up to the summation order."""
    a = dequant_mxfp4(a_packed, a_scales).astype(np.float64)
    w = dequant_mxfp4(w_packed, w_scales).astype(np.float64)
    out = (a @ w.T).astype(np.float32)
    if bias is not None:
        out = out + np.asarray(bias, np.float32)[None, :]
    return bf16_round(out)
