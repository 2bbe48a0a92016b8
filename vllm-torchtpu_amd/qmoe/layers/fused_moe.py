"""Fused-MoE entry point (the reference's `fused_moe_gmm` bridge).

Mirrors `layers/adapter/fused_moe.py:241-293` (``fused_moe_gmm``) and the
non-EP body of `layers/core/fused_moe_gmm.py:592-728` (``fused_moe_func``):
permute routes by expert, grouped GEMM gate_up with the activation fused in
its epilogue, grouped GEMM down with the routing weight fused in its epilogue
(scattering each row to its flat route slot), then the per-token sum.

Weight formats (this package's runtime layouts, produced by the MoE methods'
`process_weights_after_loading`; all N-major, K contiguous):

====================  ==========================  ====================================
format                w1 [E, 2I, H...] / w2        scales
====================  ==========================  ====================================
``mxfp4``             uint8 packed e2m1 [., ., K/2]  e8m0 uint8 [E, N, K/32]
``nvfp4``             uint8 packed e2m1 [., ., K/2]  bf16 [E, N, K/16] (fused e4m3 x global)
``int4``              int32 carriers [., ., K/8]     bf16 [E, N, K/group], group 32 / 64 / 128
                      (8 offset-binary nibbles per int32, the compressed-tensors checkpoint form)
``fp8`` / ``int8`` /  float8_e4m3fn / int8 /      f32 per-channel [E, N], or per (row, B
``e5m2``              float8_e5m2                  columns) [E, N, K/B] with B a power-of-two
                                                   multiple of 512
``fp8_w8a16``         float8_e4m3fn [E, N, K]      f32 per-(row, 128) scales [E, N, K/128]
``fp8_block``         float8_e4m3fn [E, N, K]      f32 tile scales [E, N/128, K/128]
``fp8_block_rows``    float8_e4m3fn [E, N, K]      f32 per-(row, 128) scales [E, N, K/128]
``fp8_rowquant`` /    float8_e4m3fn / int8         f32 per-channel [E, N]
``int8_rowquant``
``bf16``              bfloat16                      none
====================  ==========================  ====================================

Numeric recipe of each 1-byte format:

* ``fp8`` / ``int8`` / ``e5m2`` -- the reference's: its grouped matmul
  quantizes the activations per (row, 512 columns) in bf16 arithmetic for
  weights with quant blocks of 256+ columns (`kernels/megablox/gmm_v2.py:
  500-548`), to e4m3 for float weights (e4m3 and e5m2) and int8 for int8
  weights; the block sums are
  scaled and accumulated in f32 (the reference accumulates in bf16).
* ``fp8_w8a16`` -- the reference's for 128-column weight blocks
  (``MOE_REQUANTIZE_BLOCK_SIZE=128``): each weight is bf16(code *
  bf16(scale)), bf16 activations (`gmm_v2.py:452-462`).
* ``fp8_block`` / ``fp8_block_rows`` -- the blockwise W8A8 recipe (per
  (token, 128) e4m3 activations; BASELINE config 4's native 128x128 tiles).
* ``fp8_rowquant`` / ``int8_rowquant`` -- per-token activation quant (the
  dense linear's `kernels/quantized_matmul/util.py:80-124` recipe).

w1's N axis is ``[gate | up]`` (gate rows first), as in the reference
(`kernels/megablox/gmm_v2.py:894-901`).

The layer body is the torch custom op ``torch.ops.qmoe.fused_moe_gmm`` with a
fake implementation (output ``[T, H]`` bf16), so ``torch.compile(fullgraph=
True)`` traces through it; the reference prebuilds one custom op per static
configuration for the same reason (`layers/adapter/fused_moe.py:146-238`).
"""

from typing import Optional

import torch

from qmoe import _capi, ops
from qmoe.layers import ref_layout


MOE_FORMATS = ("mxfp4", "nvfp4", "int4", "bf16", "fp8", "int8", "e5m2", "fp8_w8a16", "fp8_block",
               "fp8_block_rows", "fp8_rowquant", "int8_rowquant", "mxfp4_mx")

# "mxfp4_mx" (opt-in, no reference counterpart): MXFP4 experts with MX
# activations -- the tokens and the intermediate quantized per 32 columns to
# e2m1 + e8m0 (`ops.mx_quant`), both GEMMs on the scaled FP4 MFMA. The
# weights are zero-padded along K at load to the MX kernel's multiple of 512
# (`linear_common.pad_mxfp4_for_mx`): w13 [E, 2I, Hp/2] + [E, 2I, Hp/32], w2
# [E, H, Ip/2] + [E, H, Ip/32]. Below MX_MOE_MIN_ROWS rows per routed expert
# (decode steps, small batches) the same numbers run on the W4A16 kernels: the
# MX activations dequantized to bf16 (exact), the unpadded weight views.
MX_MOE_MIN_ROWS = 64


def infer_weight_format(w1: torch.Tensor, w1_scale) -> str:
    if w1.dtype == torch.bfloat16:
        return "bf16"
    if w1.dtype == torch.int8:
        return "int8"
    if w1.dtype == torch.float8_e5m2:
        return "e5m2"
    if w1.dtype == torch.float8_e4m3fn:
        if w1_scale is not None and w1_scale.dim() == 3 and w1_scale.shape[-1] * 128 == w1.shape[-1]:
            return "fp8_w8a16" if w1_scale.shape[1] == w1.shape[1] else "fp8_block"
        return "fp8"
    if w1.dtype == torch.int32:
        return "int4"
    if w1.dtype == torch.uint8 or "float4" in str(w1.dtype):
        return "nvfp4" if w1_scale is not None and w1_scale.dtype == torch.bfloat16 else "mxfp4"
    raise ValueError(f"unsupported MoE weight dtype {w1.dtype}")


def _per_channel(s, E, N) -> bool:
    return (s is not None and s.dtype == torch.float32 and s.shape[0] == E and s.shape[1] == N
            and (s.dim() == 2 or (s.dim() == 3 and s.shape[2] == 1)))


def can_use_dense_expert(hidden_states, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, activation, fmt) -> bool:
    """Admission of the dense-expert decode branch
    (`kernels/experimental/moe_dense_expert.py:50-90`, ``can_use_dense_expert``),
    on this package's expert layout: silu; per-channel e4m3 experts (format
    ``fp8``: w1 [E, 2I, H], w2 [E, H, I], f32 scales [E, 2I] / [E, H], or
    [E, N, 1]); no biases; bf16 tokens; T % 16 == 0, H % 512 == 0, I % 128 == 0.
    The reference's hardware clause (native FP8 and a 512-column activation
    block at least one matrix-unit column wide) always holds here: per-channel
    experts always quantize their activations per (row, 512)."""
    if activation != "silu" or fmt != "fp8" or w1_bias is not None or w2_bias is not None:
        return False
    if hidden_states.dim() != 2 or w1.dim() != 3 or w2.dim() != 3 or hidden_states.dtype != torch.bfloat16:
        return False
    if w1.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
        return False
    m, h = hidden_states.shape
    e, out, i = w2.shape
    if min(m, h, i, e) <= 0 or m % 16 or h % 512 or i % 128:
        return False
    if out != h or tuple(w1.shape) != (e, 2 * i, h):
        return False
    return _per_channel(w1_scale, e, 2 * i) and _per_channel(w2_scale, e, h)


def merge_repeated_routes(topk_weights: torch.Tensor, topk_ids: torch.Tensor):
    """The dense-expert branch's coefficient table in route form
    (`kernels/experimental/moe_dense_expert.py:258-268`): a token's
    coefficient for an expert is the float32 sum, in route order, of the
    weights of its routes to that expert. The first of those routes carries
    the sum (rounded to the routing weights' bf16, the grouped path's
    coefficient dtype) and the later ones become invalid (id -1), so weights
    +w and -w on one expert cancel to exactly 0 and the zero-coefficient
    mask drops the expert even when its output is not finite. Returns
    (weights, ids) of the same shapes."""
    ids = topk_ids.to(torch.int32)
    w = topk_weights.float()
    k = ids.shape[1]
    same = ids[:, :, None] == ids[:, None, :]  # [T, k, k]: route i and route j name one expert
    coeff = torch.zeros_like(w)
    for j in range(k):  # the reference's accumulation order
        coeff = coeff + torch.where(same[:, :, j], w[:, j:j + 1], torch.zeros_like(w))
    earlier = torch.ones((k, k), dtype=torch.bool, device=ids.device).tril(-1)  # [i, j]: j < i
    repeat = (same & earlier).any(-1)
    merged_ids = torch.where(repeat, torch.full_like(ids, -1), ids)
    merged_w = torch.where(repeat, torch.zeros_like(coeff), coeff).to(torch.bfloat16)
    return merged_w, merged_ids


def _dense_expert_admitted(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, activation, fmt) -> bool:
    """``0 < T <= TPU_MOE_DENSE_EXPERT_THRESHOLD`` and the admission rule, the
    token threshold first (`layers/core/fused_moe_gmm.py:669-686`)."""
    from qmoe import envs

    return (0 < x.shape[0] <= envs.TPU_MOE_DENSE_EXPERT_THRESHOLD
            and can_use_dense_expert(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, activation, fmt))


def fused_moe_gmm(hidden_states, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, topk_weights,
                  topk_ids, experts_start, topk, activation, rhs_quant_dtype=None,
                  skip_padded_tokens=None, weight_format=None):
    """Routed-expert MoE forward (`fused_moe.py:241-293`). Returns bf16 [T, H].

    ``experts_start`` is the reference's expert-parallel offset; this build
    runs the whole expert set on one GPU, so it must be None or 0.
    ``rhs_quant_dtype``: ``int4`` (any dtype object or string naming int4) marks
    packed-int4 int32 weights (`compressed_tensors_moe_w4a16.py:380-405`).

    Weights come in this package's layouts (table above; what the MoE
    methods hold) or in the reference's runtime layout -- ``w1 [E, H, 2I]``,
    ``w2 [E, I, H]``, scales ``[E, K/B, 1, N]`` or ``[E, K/B, N]``, biases
    ``[E, 1, N]`` -- which is recognized from the shapes and repacked once
    per weight tensor (`qmoe/layers/ref_layout.py`).
    """
    # The reference passes experts_start as a 0-d int32 tensor exactly when
    # expert parallelism is on (`layers/adapter/fused_moe.py:241-293`); this
    # build holds the whole expert set, so any tensor (whatever its value) and
    # any non-zero offset is refused rather than silently ignored.
    if experts_start is not None and (isinstance(experts_start, torch.Tensor) or int(experts_start) != 0):
        raise NotImplementedError("expert parallelism is out of scope: experts_start must be None or 0")
    if rhs_quant_dtype is not None:
        if "int4" not in str(rhs_quant_dtype):
            raise NotImplementedError(f"rhs_quant_dtype {rhs_quant_dtype} is not supported (int4 only)")
        weight_format = weight_format or "int4"
    if weight_format is None and ref_layout.is_reference_moe_layout(hidden_states.shape[-1], w1, w2, w1_scale):
        # the reference's runtime layout (K-major, [E, K/B, 1, N] scales),
        # repacked once per weight tensor
        w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, weight_format = ref_layout.moe_weights(
            hidden_states.shape[-1], w1, w2, w1_scale, w2_scale, w1_bias, w2_bias)
    fmt = weight_format or infer_weight_format(w1, w1_scale)
    if fmt not in MOE_FORMATS:
        raise ValueError(f"unknown MoE weight format {fmt!r}")
    ops.act_code(activation)  # NotImplementedError for an unknown activation string
    T, H = hidden_states.shape
    if topk_weights.shape != (T, topk) or topk_ids.shape != (T, topk):
        raise ValueError(f"topk tensors must be [{T}, {topk}]")
    # The dense-expert decode branch (`fused_moe_gmm.py:669-686`) weighs each
    # active expert's output by the token's summed routing coefficient and
    # masks zero coefficients before accumulating (`moe_dense_expert.py:
    # 175-181`), so a zero-weight route contributes exactly 0 even when its
    # expert's output is not finite. Its activation recipe is already this
    # format's (per (row, 512) bf16-arithmetic e4m3 codes), and the grouped
    # path visits each active expert's weights once, as it does; what it
    # adds is the coefficient table (a token's repeated routes to one expert
    # merged into one coefficient) and the mask, which is the skipping of
    # zero-coefficient routes.
    if _dense_expert_admitted(hidden_states, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, activation, fmt):
        skip_padded_tokens = True
        topk_weights, topk_ids = merge_repeated_routes(topk_weights, topk_ids)
    x = hidden_states if hidden_states.dtype == torch.bfloat16 else hidden_states.to(torch.bfloat16)
    # `fused_moe_gmm.py:653`: routing weights take the hidden dtype
    tw = topk_weights.to(torch.bfloat16)
    ids = topk_ids.to(torch.int32)
    return torch.ops.qmoe.fused_moe_gmm(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, tw, ids, int(topk),
                                        activation or "", bool(skip_padded_tokens), fmt)


@torch.library.custom_op("qmoe::fused_moe_gmm", mutates_args=())
def _fused_moe_gmm_op(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w1_scale: Optional[torch.Tensor],
                      w2_scale: Optional[torch.Tensor], w1_bias: Optional[torch.Tensor],
                      w2_bias: Optional[torch.Tensor], tw: torch.Tensor, topk_ids: torch.Tensor, topk: int,
                      activation: str, skip: bool, fmt: str) -> torch.Tensor:
    """Checked operands: x bf16 [T, H]; tw bf16 / topk_ids int32 [T, topk]."""
    tw = tw.contiguous()
    meta = ops.moe_dispatch(topk_ids, tw, w1.shape[0], skip)
    return _moe_body(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, tw, topk_ids, topk, activation, skip, fmt,
                     meta)


@torch.library.custom_op("qmoe::routed_moe", mutates_args=())
def _routed_moe_op(x: torch.Tensor, router_logits: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                   w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor],
                   w1_bias: Optional[torch.Tensor], w2_bias: Optional[torch.Tensor], topk: int, scoring_func: str,
                   renormalize: bool, e_bias: Optional[torch.Tensor], routed_scaling_factor: float,
                   num_expert_group: int, topk_group: int, activation: str, skip: bool,
                   fmt: str) -> torch.Tensor:
    """Decode-size layer (1..16 tokens, at most 64 routes): routing and
    dispatch in one launch (`qmoe_moe_route_dispatch`), then the experts."""
    tw, ids, meta = ops.moe_route_dispatch(router_logits, topk, scoring_func, renormalize, e_bias,
                                           routed_scaling_factor, num_expert_group, topk_group, skip)
    return _moe_body(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, tw, ids, topk, activation, skip, fmt, meta)


@_routed_moe_op.register_fake
def _(x, router_logits, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, topk, scoring_func, renormalize, e_bias,
      routed_scaling_factor, num_expert_group, topk_group, activation, skip, fmt):
    return x.new_empty(x.shape, dtype=torch.bfloat16)


def moe_forward(layer, x, router_logits, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, weight_format,
                skip_padded_tokens=None, input_ids=None):
    """Routing + routed experts of a MoE method's `apply_monolithic`
    (`layers/adapter/quantization/fp8.py:1108-1222`: route, then
    `fused_moe_gmm`). A decode-size batch (1..16 bf16 tokens, at most 64
    routes) with the layer's own scoring takes the fused route + dispatch
    launch; anything else (a model-supplied routing function, hash routing,
    larger batches) routes first and calls `fused_moe_gmm`."""
    from qmoe.layers import moe_routing

    topk = layer.moe_config.experts_per_token
    T = x.shape[0]
    custom = getattr(layer, "custom_routing_function", None)
    hashed = getattr(layer, "hash_indices_table", None) is not None and input_ids is not None
    act = layer._qmoe_activation
    fusable = (custom is None and not hashed and x.dtype == torch.bfloat16
               and 1 <= T <= ops.ROUTE_DISPATCH_MAX_TOKENS and T * topk <= ops.ROUTE_DISPATCH_MAX_ROUTES
               and w1.shape[0] <= 512 and layer.scoring_func in ops._SCORING)
    if not fusable:
        topk_weights, topk_ids = moe_routing.route(layer, x, router_logits, input_ids=input_ids)
        return fused_moe_gmm(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, topk_weights, topk_ids, None, topk,
                             act, skip_padded_tokens=skip_padded_tokens, weight_format=weight_format)
    ops.act_code(act)
    if _dense_expert_admitted(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, act, weight_format):
        skip_padded_tokens = True  # the dense-expert branch's coefficient mask, as in fused_moe_gmm
    bias, rsf, ng, tg = moe_routing.routing_params(layer)
    return torch.ops.qmoe.routed_moe(x, router_logits, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, int(topk),
                                     layer.scoring_func, bool(layer.renormalize), bias, float(rsf), int(ng),
                                     int(tg), act or "", bool(skip_padded_tokens), weight_format)


def _gmm_scale(s, E):
    """Weight scales of the grouped-matmul recipe: per-channel [E, N] or per
    (row, B columns) [E, N, K/B], f32, contiguous."""
    s = s.float()
    if s.dim() == 3 and s.shape[-1] == 1:
        s = s[..., 0]
    return s.reshape(E, *s.shape[1:]).contiguous()


def _moe_body(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, tw, topk_ids, topk, activation, skip, fmt, meta):
    """The experts of a routed layer, given the dispatch metadata."""
    activation = activation or None
    T, H = x.shape
    E = w1.shape[0]
    x = x.contiguous()
    M = T * topk
    common = dict(group_offs=meta["group_offs"], active=meta["active"],
                  num_active=meta["num_active"], slots=E, max_rows=T, M=M)

    b1 = w1_bias.float().reshape(E, -1).contiguous() if w1_bias is not None else None
    b2 = w2_bias.float().reshape(E, -1).contiguous() if w2_bias is not None else None
    u8 = lambda t: t.view(torch.uint8)  # noqa: E731

    if fmt == "mxfp4_mx":
        Hp, Ip = w1.shape[-1] * 2, w2.shape[-1] * 2
        I = w1.shape[1] // 2 if activation else w1.shape[1]
        if M >= MX_MOE_MIN_ROWS * min(E, M):
            xq, xs = ops.mx_quant(x, k_pad=Hp)
            inter = ops.gemm(_capi.W4A4_MX, xq, u8(w1), a_scale=xs, w_scale=u8(w1_scale), bias=b1,
                             a_rows=meta["token_sorted"], activation=activation, **common)
            a2, a2_scale = ops.mx_quant(inter, k_pad=Ip)
            kind, wf, bn = _capi.W4A4_MX, 0, 1
            w2k, w2s = u8(w2), u8(w2_scale)
        else:
            xd = ops.mx_quant(x, codes=False, dequantized=True)
            inter = ops.gemm(_capi.W4A16_MX, xd, u8(w1)[..., : H // 2], w_scale=u8(w1_scale)[..., : H // 32],
                             bias=b1, a_rows=meta["token_sorted"], activation=activation, **common)
            a2 = ops.mx_quant(inter, codes=False, dequantized=True)
            a2_scale, kind, wf, bn = None, _capi.W4A16_MX, 0, 1
            w2k, w2s = u8(w2)[..., : I // 2], u8(w2_scale)[..., : I // 32]
    elif fmt in ("mxfp4", "nvfp4", "int4"):
        kind = {"mxfp4": _capi.W4A16_MX, "nvfp4": _capi.W4A16_NV, "int4": _capi.W4A16_I4}[fmt]
        sc = u8 if fmt == "mxfp4" else (lambda t: t)  # noqa: E731
        inter = ops.gemm(kind, x, u8(w1), w_scale=sc(w1_scale), bias=b1,
                         a_rows=meta["token_sorted"], activation=activation, **common)
        a2, a2_scale, wf, bn = inter, None, 0, 1
        w2k, w2s = u8(w2), sc(w2_scale)
    elif fmt == "bf16":
        inter = ops.gemm(_capi.W16A16, x, w1, bias=b1, a_rows=meta["token_sorted"],
                         activation=activation, **common)
        a2, a2_scale, kind, wf, bn = inter, None, _capi.W16A16, 0, 1
        w2k, w2s = w2, None
    elif fmt in ("fp8_block", "fp8_block_rows"):
        bn = 128 if fmt == "fp8_block" else 1
        xq, xs = ops.row_quant(x, "fp8", block=128)
        inter = ops.gemm(_capi.W8A8_BLK, u8(xq), u8(w1), a_scale=xs, w_scale=w1_scale, ws_bn=bn,
                         bias=b1, a_rows=meta["token_sorted"], activation=activation, **common)
        a2q, a2_scale = ops.row_quant(inter, "fp8", block=128)
        a2, kind, wf = u8(a2q), _capi.W8A8_BLK, 0
        w2k, w2s = u8(w2), w2_scale
    elif fmt in ("fp8", "int8", "e5m2"):
        # the reference's grouped-matmul recipe: per-(row, 512) bf16-arithmetic
        # activation quant before each GEMM (e4m3 for float experts, e5m2
        # included: `kernels/megablox/gmm_v2.py:1199-1215`)
        qd, wf = {"fp8": ("fp8", 0), "int8": ("int8", 1), "e5m2": ("fp8", 2)}[fmt]
        xq, xs = ops.row_quant(x, qd, mode="gmm")
        inter = ops.gemm(_capi.W8A8_GMM, u8(xq), u8(w1), a_scale=xs, w_scale=_gmm_scale(w1_scale, E),
                         wfmt=wf, bias=b1, a_rows=meta["token_sorted"], activation=activation, **common)
        a2q, a2_scale = ops.row_quant(inter, qd, mode="gmm")
        a2, kind, bn = u8(a2q), _capi.W8A8_GMM, 1
        w2k, w2s = u8(w2), _gmm_scale(w2_scale, E)
    elif fmt == "fp8_w8a16":
        inter = ops.gemm(_capi.W8A16_BLK, x, u8(w1), w_scale=w1_scale.float().contiguous(), ws_bn=1, bias=b1,
                         a_rows=meta["token_sorted"], activation=activation, **common)
        a2, a2_scale, kind, wf, bn = inter, None, _capi.W8A16_BLK, 0, 1
        w2k, w2s = u8(w2), w2_scale.float().contiguous()
    elif fmt in ("fp8_rowquant", "int8_rowquant"):
        qd, wf = ("fp8", 0) if fmt == "fp8_rowquant" else ("int8", 1)
        xq, xs = ops.row_quant(x, qd)
        inter = ops.gemm(_capi.W8A8_PC, u8(xq), u8(w1), a_scale=xs,
                         w_scale=w1_scale.float().reshape(E, -1).contiguous(), wfmt=wf, bias=b1,
                         a_rows=meta["token_sorted"], activation=activation, **common)
        a2q, a2_scale = ops.row_quant(inter, qd)
        a2, kind, bn = u8(a2q), _capi.W8A8_PC, 1
        w2k, w2s = u8(w2), w2_scale.float().reshape(E, -1).contiguous()
    else:
        raise ValueError(f"unknown MoE weight format {fmt!r}")

    routed = torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
    ops.gemm(kind, a2, w2k, a_scale=a2_scale, w_scale=w2s, wfmt=wf, ws_bn=bn, bias=b2,
             row_weight=meta["sorted_weight"], y_rows=meta["sorted_idx"], out=routed, **common)
    return ops.moe_combine(routed, topk_ids, tw, E, skip)


@_fused_moe_gmm_op.register_fake
def _(x, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias, tw, topk_ids, topk, activation, skip, fmt):
    return x.new_empty(x.shape, dtype=torch.bfloat16)
