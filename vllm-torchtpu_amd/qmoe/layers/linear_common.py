"""Dense quantized-matmul entry points (the reference's `linear_common`).

Mirrors `layers/adapter/linear_common.py` of the reference plugin:
``quantized_matmul(x, w_q, w_s, w8a16_max_rows=0)`` (`:162-185`, dispatch
`:69-128`) and ``quantized_matmul_fp4(x, w_q, w_s)`` (`:242-255`). Same
argument meaning and the same ValueError texts; the computation runs in the
qmoe HIP kernels.

Both are registered as torch custom ops (``torch.ops.qmoe.quantized_matmul``
and ``torch.ops.qmoe.quantized_matmul_fp4``) with fake implementations, so a
model that calls them compiles with ``torch.compile(fullgraph=True)`` (the
reference builds its ops the same way: custom ops with ``register_fake``,
`linear_common.py:131-159`). Shape and layout checks run in the Python
wrappers below, before the op, so they raise at trace time too.

Weight layout: the reference's runtime weight is the canonical (k, n)
``[n_in, n_out]`` array. Here ``w_q`` has that same logical shape but must be
the transposed VIEW of an N-major ``[n_out, n_in]`` buffer (stride
``(1, n_in)``), which is what this package's `process_weights_after_loading`
produces: each output channel's K values stay contiguous for 16-byte HBM
loads. A K-major contiguous ``[n_in, n_out]`` tensor is rejected rather than
transposed per call.
"""

from typing import Optional

import torch

from qmoe import _capi, ops
from qmoe.layers import ref_layout

# Markers of the reference's linear layers (`linear_common.py:30-53`). A
# module that reads a linear layer's ``.weight`` raw sets KEEP_VLLM_LAYOUT on
# it so the weight keeps vLLM's ``[n_out, n_in]`` layout; the reference
# flips every other weight to ``[n_in, n_out]`` once and records that with
# WEIGHT_FLIPPED. This package keeps every weight in ``[n_out, n_in]`` (the
# kernels read N-major weights), so both hold trivially: raw readers always
# see vLLM's layout and no flip can be repeated.
KEEP_VLLM_LAYOUT_ATTR = "_tpu_keep_vllm_weight_layout"
WEIGHT_FLIPPED_ATTR = "_tpu_weight_flipped"


def _weight_nk(w_q: torch.Tensor) -> torch.Tensor:
    """[K, N] logical weight -> the N-major [N, K] buffer it views (this
    package's layout: ``weight.t()`` of the ``[n_out, n_in]`` parameter). A
    contiguous K-major ``[n_in, n_out]`` weight (the reference's runtime
    layout after its load-time flip, `fp8.py:1598-1617`) is transposed into
    an N-major copy once per weight tensor (`qmoe/layers/ref_layout.py`)."""
    if w_q.dim() != 2:
        raise ValueError(f"weight must be 2-D [n_in, n_out], got {tuple(w_q.shape)}")
    w_nk = w_q.t()
    if not w_nk.is_contiguous():
        w_nk = ref_layout.nmajor_copy(w_q)
    return w_nk


# numeric regimes of `quantized_matmul` (the custom op's `regime` argument)
REGIME_PER_CHANNEL = 0  # `util.py:80-124`: per-token activation quant, per-channel weights
REGIME_NATIVE_BLOCKS = 1  # this build's 128x128-tile form: per-(token, 128) activation quant
REGIME_GMM_QUANT_LHS = 2  # gmm_v2, weight blocks >= 256: per-(token, 512) bf16-arithmetic quant
REGIME_GMM_W8A16 = 3  # gmm_v2, weight blocks < 256: bf16(code * bf16(scale)) weights, bf16 x

# quant blocks below this many columns are dequantized before the matmul
# (the reference's MXU width, `kernels/megablox/gmm_v2.py:255-262`)
GMM_DEQUANT_BEFORE_BELOW = 256


def _rank4_blocks(w_s: torch.Tensor, k_dim: int, n_out: int):
    """The reference's rank-4 ``[1, K/B, 1, N]`` scale (validated with its
    messages, `linear_common.py:83-104`) -> (``[N, K/B]`` f32 view or copy,
    B). A rank-4 view of an N-major ``[N, K/B]`` buffer (what this package's
    `process_weights_after_loading` stores) needs no copy."""
    _, sharded_num_blocks, mid, scale_n_out = w_s.shape
    if mid != 1:
        raise ValueError(f"Blockwise weight scale axis 2 must be 1, got {w_s.shape=}")
    if scale_n_out != n_out:
        raise ValueError(
            f"Blockwise weight scale output dim {scale_n_out} must match "
            f"weight output dim {n_out}."
        )
    if sharded_num_blocks <= 0 or k_dim % sharded_num_blocks != 0:
        raise ValueError(
            f"Input hidden dim {k_dim} must be divisible by block scale "
            f"count {sharded_num_blocks}."
        )
    sc = w_s[0, :, 0, :].t()
    if sc.dtype != torch.float32 or not sc.is_contiguous():
        sc = sc.float().contiguous()
    return sc, k_dim // sharded_num_blocks


def _native_blocks(w_s: torch.Tensor, k_dim: int, n_out: int):
    """This build's compact block-scale form -> (f32 [N/bn, K/128], bn):
    per (channel, 128-column block) (bn = 1) or per 128x128 tile (bn = 128)."""
    if w_s.shape[1] * 128 != k_dim:
        raise ValueError(f"block scale has {w_s.shape[1]} K blocks, expected {k_dim // 128}")
    if w_s.shape[0] == n_out:
        return w_s.float().contiguous(), 1
    if w_s.shape[0] == (n_out + 127) // 128:
        return w_s.float().contiguous(), 128
    raise ValueError(f"block scale rows {w_s.shape[0]} match neither {n_out} nor {n_out // 128}")


def quantized_matmul(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor,
                     w8a16_max_rows: int = 0) -> torch.Tensor:
    """Runtime quantized dense linear, `linear_common.py:162-185` + `:69-128`.

    * ``w_s`` 1-D ``[n_out]``: per-channel (`kernels/quantized_matmul/util.py:
      80-124`). e4m3 weights with ``0 < rows <= w8a16_max_rows`` keep bf16
      activations (W8A16); otherwise activations are quantized per token (e4m3
      in f32 / int8 in bf16 arithmetic) -- W8A8.
    * ``w_s`` rank-4 ``[1, K/B, 1, N]`` (the reference's blockwise runtime
      layout): the single-group grouped matmul of `:88-114`, in its regime for
      B (`kernels/megablox/gmm_v2.py:255-262, 452-548`): B < 256 (B = 128):
      e4m3 weights dequantized to bf16(code * bf16(scale)), bf16 activations;
      B >= 256 (B = K, or a power-of-two multiple of 512): activations
      quantized per (token, 512 columns) in bf16 arithmetic to e4m3 (int8 for
      int8 weights), f32 accumulation of the scaled block sums.
    * ``w_s`` 2-D ``[N/bn, K/128]`` (this build's native 128x128-tile form,
      bn = 128, or per-(channel, 128) with bn = 1): activations quantized per
      (token, 128 columns) in f32, the blockwise W8A8 recipe of
      `kernels/quantized_matmul/blockwise_kernel.py:197-247`.
    """
    if x.shape[-1] != w_q.shape[0]:
        raise ValueError(
            f"Input hidden dim {x.shape[-1]} must match weight hidden dim "
            f"{w_q.shape[0]}."
        )
    orig_out_shape = (*x.shape[:-1], w_q.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    w_nk = _weight_nk(w_q)
    k_dim, n_out = w_q.shape
    if w_nk.dtype not in (torch.int8, torch.float8_e4m3fn, torch.float8_e5m2):
        raise ValueError(f"Unsupported quantized dtype: {w_nk.dtype}")
    if w_s.dim() == 1:
        if w_s.shape[0] != n_out:
            raise ValueError(f"per-channel scale has {w_s.shape[0]} entries, expected {n_out}")
        regime = REGIME_PER_CHANNEL
    elif w_s.dim() == 4:
        w_s, block = _rank4_blocks(w_s, k_dim, n_out)
        if block < GMM_DEQUANT_BEFORE_BELOW:
            if block != 128 or w_nk.dtype != torch.float8_e4m3fn:
                raise NotImplementedError(
                    f"qmoe dequantizes weight blocks under {GMM_DEQUANT_BEFORE_BELOW} columns for "
                    f"float8_e4m3fn weights with 128-column blocks only, got {w_nk.dtype} blocks of {block}")
            regime = REGIME_GMM_W8A16
        else:
            if block != k_dim and (block % 512 or (block // 512) & (block // 512 - 1)):
                raise NotImplementedError(
                    f"qmoe runs weight blocks of 256+ columns as per-channel (B = K) or power-of-two "
                    f"multiples of 512 columns, got {block} for K={k_dim}")
            if k_dim % 128:
                raise NotImplementedError(f"the quantized-lhs regime needs K % 128 == 0, got {k_dim}")
            regime = REGIME_GMM_QUANT_LHS
    elif w_s.dim() == 2:
        if w_nk.dtype != torch.float8_e4m3fn:
            raise ValueError(f"blockwise kernels take float8_e4m3fn weights, got {w_nk.dtype}")
        w_s, _ = _native_blocks(w_s, k_dim, n_out)
        regime = REGIME_NATIVE_BLOCKS
    else:
        raise ValueError(f"unsupported weight scale shape {tuple(w_s.shape)}")
    out = torch.ops.qmoe.quantized_matmul(x2, w_nk, w_s, int(w8a16_max_rows), regime)
    return out.reshape(orig_out_shape)


@torch.library.custom_op("qmoe::quantized_matmul", mutates_args=())
def _quantized_matmul_op(x2: torch.Tensor, w_nk: torch.Tensor, w_s: torch.Tensor,
                         w8a16_max_rows: int, regime: int) -> torch.Tensor:
    """Checked operands: x2 bf16 [rows, K]; w_nk N-major [N, K] codes; w_s
    per-channel f32 [N], [N, K/B] (the gmm_v2 regimes) or compact native
    block scales [N/bn, K/128]."""
    n_out, k_dim = w_nk.shape
    rows = x2.shape[0]
    wq = w_nk.view(torch.uint8)
    is_int = w_nk.dtype == torch.int8
    # weight code format of the W8A8 kinds: 0 e4m3, 1 int8, 2 e5m2
    wfmt = 1 if is_int else (2 if w_nk.dtype == torch.float8_e5m2 else 0)
    if regime == REGIME_PER_CHANNEL:
        ws = w_s.float().contiguous()
        if not is_int and 0 < rows <= w8a16_max_rows:
            if wfmt == 2:
                raise NotImplementedError("qmoe runs W8A16 (w8a16_max_rows) for float8_e4m3fn weights only")
            return ops.gemm(_capi.W8A16_PC, x2, wq, w_scale=ws)
        # per-token activation quant (to the weight dtype, `util.py:108`) +
        # W8A8 in one call (decode sizes quantize inside the streaming
        # kernel; larger ones quantize first)
        x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            x2 = x2.clone()
        return ops.gemm(_capi.W8A8_PC_DYN, x2, wq, w_scale=ws, wfmt=wfmt)
    if regime == REGIME_GMM_W8A16:
        return ops.gemm(_capi.W8A16_BLK, x2, wq, w_scale=w_s, ws_bn=1)
    if regime == REGIME_GMM_QUANT_LHS:
        # e4m3 activations for any float weights (`kernels/megablox/gmm_v2.py:1199-1215`)
        xq, xs = ops.row_quant(x2, "int8" if is_int else "fp8", mode="gmm")
        return ops.gemm(_capi.W8A8_GMM, xq.view(torch.uint8), wq, a_scale=xs, w_scale=w_s, wfmt=wfmt)
    sb, bn = _native_blocks(w_s, k_dim, n_out)
    xq, xs = ops.row_quant(x2, "fp8", block=128)
    return ops.gemm(_capi.W8A8_BLK, xq.view(torch.uint8), wq, a_scale=xs, w_scale=sb, ws_bn=bn)


@_quantized_matmul_op.register_fake
def _(x2, w_nk, w_s, w8a16_max_rows, regime):
    return x2.new_empty((x2.shape[0], w_nk.shape[0]), dtype=torch.bfloat16)


def quantized_matmul_fp4(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor,
                         bias: torch.Tensor | None = None) -> torch.Tensor:
    """FP4 W4A16 dense linear, `linear_common.py:188-209, 242-255`.

    ``w_q``: packed e2m1 codes, N-major ``[n_out, n_in/2]`` uint8 (the
    checkpoint layout; low nibble = even k), or the reference's runtime form
    (K-major ``float4_e2m1fn_x2`` / uint8 ``[n_in, n_out/2]`` with a rank-4
    ``[1, n_in/B, 1, n_out]`` float32 scale, B = 16 or 32), repacked once per
    weight tensor (`qmoe/layers/ref_layout.py`). ``w_s`` picks the format:
    e8m0 bytes ``[n_out, n_in/32]`` (MXFP4), or bf16 / f32 block scales
    ``[n_out, n_in/16]`` (NVFP4: the fused e4m3 x global scale; f32 values are
    rounded to bf16, which is what the reference's in-kernel dequantization
    does with them, `kernels/megablox/gmm_v2.py:452-462`). bf16 activations
    stay unquantized (both blocks are below the reference's
    dequantize-after-matmul threshold), f32 accumulate.
    """
    if w_s.dim() == 4:
        # the reference's runtime layout: K-major fp4 [n_in, n_out] (bytes
        # [n_in, n_out / 2]) + [1, n_in / B, 1, n_out] float32, repacked once
        w_q, w_s = ref_layout.fp4_linear(w_q, w_s, x.shape[-1])
    nv = w_s.dtype in (torch.bfloat16, torch.float32)
    blk = 16 if nv else 32
    if w_q.dim() != 2 or w_s.dim() != 2:
        raise ValueError(f"quantized_matmul_fp4 expects w_q [n_out, n_in/2] and w_s [n_out, n_in/{blk}]")
    n_out = w_s.shape[0]
    k_dim = x.shape[-1]
    if w_q.shape != (n_out, k_dim // 2) or w_s.shape[1] * blk != k_dim:
        raise ValueError(
            f"{'NVFP4' if nv else 'MXFP4'} weight {tuple(w_q.shape)} / scale {tuple(w_s.shape)} "
            f"do not match input dim {k_dim}"
        )
    x2 = x.reshape(-1, k_dim)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    w_s = w_s.to(torch.bfloat16) if nv else w_s.view(torch.uint8)
    out = torch.ops.qmoe.quantized_matmul_fp4(x2, w_q.view(torch.uint8), w_s, bias)
    return out.reshape(*x.shape[:-1], n_out)


@torch.library.custom_op("qmoe::quantized_matmul_fp4", mutates_args=())
def _quantized_matmul_fp4_op(x2: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor,
                             bias: Optional[torch.Tensor]) -> torch.Tensor:
    kind = _capi.W4A16_NV if w_s.dtype == torch.bfloat16 else _capi.W4A16_MX
    return ops.gemm(kind, x2, w_q.contiguous(), w_scale=w_s.contiguous(), bias=bias)


@_quantized_matmul_fp4_op.register_fake
def _(x2, w_q, w_s, bias):
    return x2.new_empty((x2.shape[0], w_s.shape[0]), dtype=torch.bfloat16)


# ---------------------------------------------------------------- opt-in MX activations (W4A4)
#
# No counterpart in the reference (its W4A4 MXFP4 method runs bf16
# activations, `compressed_tensors_moe_w4an_mxfp4.py:49-55`): MXFP4 weights
# with activations quantized per 32 columns to e2m1 + e8m0 (`ops.mx_quant`,
# the reference's ue8m0 block rule and e2m1 encoder), both scales applied by
# the MFMA. The MX kernel takes K in multiples of 512 (at least 1024), so
# the weight is zero-padded along K once at load (`pad_mxfp4_for_mx`).
# Problems too small to fill the CUs with 256 x 256 tiles run the same
# numbers on the bf16-activation kernels: the MX-quantized activations are
# exact in bf16 and the products of the two formats are exact in f32, so
# only the f32 summation order differs.

MX_K_ALIGN = 512
# 256 x 256 tiles below which the bf16-activation kernels take the problem
MX_MIN_TILES = 128


def mx_padded_k(k: int) -> int:
    """K of the MX kernel for a layer of input size ``k``: a multiple of 512,
    at least 1024."""
    return max(2 * MX_K_ALIGN, -(-int(k) // MX_K_ALIGN) * MX_K_ALIGN)


def pad_mxfp4_for_mx(w_q: torch.Tensor, w_s: torch.Tensor):
    """Zero-pad MXFP4 weights ``[n_out, k/2]`` codes + ``[n_out, k/32]`` e8m0
    along K to ``mx_padded_k(k)``: codes 0 (and scale byte 127, 1.0) in the
    padding, so the extra products are zero."""
    n, kb = w_q.shape
    k = 2 * kb
    if w_s.shape != (n, k // 32):
        raise ValueError(f"MXFP4 scale {tuple(w_s.shape)} does not match codes {tuple(w_q.shape)}")
    kp = mx_padded_k(k)
    wq = torch.zeros((n, kp // 2), dtype=torch.uint8, device=w_q.device)
    ws = torch.full((n, kp // 32), 127, dtype=torch.uint8, device=w_s.device)
    wq[:, :kb] = w_q.view(torch.uint8)
    ws[:, : k // 32] = w_s.view(torch.uint8)
    return wq, ws


def quantized_matmul_mxfp4_a4(x: torch.Tensor, w_pad: torch.Tensor, ws_pad: torch.Tensor, k: int,
                              bias: torch.Tensor | None = None) -> torch.Tensor:
    """MXFP4 weight x MX-quantized activation linear: ``x`` [..., k] (bf16 or
    castable), ``w_pad`` / ``ws_pad`` from `pad_mxfp4_for_mx`, optional bias
    [n_out] added in f32 before the bf16 rounding. bf16 out."""
    n_out = w_pad.shape[0]
    kp = w_pad.shape[1] * 2
    if x.shape[-1] != k or k % 32 or kp != mx_padded_k(k) or ws_pad.shape != (n_out, kp // 32):
        raise ValueError(f"MX linear: input dim {x.shape[-1]}, k {k}, padded weight {tuple(w_pad.shape)} / "
                         f"{tuple(ws_pad.shape)} do not match")
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    b = None if bias is None else bias.reshape(n_out).to(torch.float32)
    out = torch.ops.qmoe.quantized_matmul_mxfp4_a4(x2, w_pad, ws_pad, b)
    return out.reshape(*x.shape[:-1], n_out)


@torch.library.custom_op("qmoe::quantized_matmul_mxfp4_a4", mutates_args=())
def _quantized_matmul_mxfp4_a4_op(x2: torch.Tensor, w_pad: torch.Tensor, ws_pad: torch.Tensor,
                                  bias: Optional[torch.Tensor]) -> torch.Tensor:
    M, k = x2.shape
    n_out, kp = w_pad.shape[0], w_pad.shape[1] * 2
    if -(-M // 256) * -(-n_out // 256) >= MX_MIN_TILES:
        q, sc = ops.mx_quant(x2, k_pad=kp)
        return ops.gemm(_capi.W4A4_MX, q, w_pad, a_scale=sc, w_scale=ws_pad, bias=bias)
    xq = ops.mx_quant(x2, codes=False, dequantized=True)
    return ops.gemm(_capi.W4A16_MX, xq, w_pad[:, : k // 2], w_scale=ws_pad[:, : k // 32], bias=bias)


@_quantized_matmul_mxfp4_a4_op.register_fake
def _(x2, w_pad, ws_pad, bias):
    return x2.new_empty((x2.shape[0], w_pad.shape[0]), dtype=torch.bfloat16)
