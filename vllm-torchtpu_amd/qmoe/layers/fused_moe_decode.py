"""Serve a MoE layer's decode steps with the fused decode MoE op (shared
expert + routed experts in one call), `layers/adapter/fused_moe_decode.py`
of the reference on one GPU.

Arming (`arm_fused_moe_decode`, once after load, with
``FUSED_MOE_DECODE_KERNEL=1``) takes the MoE runners whose routed layer is
served by `Fp8MoEMethod` with silu experts and no biases, and whose shared
expert is an FP8 MLP (gate_up_proj -> SiluAndMul -> down_proj, optionally
gated by a one-output ``expert_gate`` linear). The shared expert's tensors
become non-persistent buffers of the routed layer, the runner is told it
has no shared expert, and its ``routed_scaling_factor`` moves into the op
(which scales the routed experts only) as the reference does
(`fused_moe_decode.py:513-619`).

An armed layer's forward (`fused_moe_decode`) runs `ops.moe_decode` for
steps of up to ``FUSED_MOE_DECODE_KERNEL_MAX_TOKENS`` tokens (capped at the
kernel's 64) -- `fused_moe_decode_routed` with the routing folded into the
op when the layer uses the plain or grouped rule -- and above that what the
runner would compute with the op off:
the GMM MoE path, the shared expert's linears and their sum
(`fused_moe_decode.py:105-164`, `_gmm_layer`). One GPU: there is no
all-reduce and no expert parallelism.

Weights stay in the layouts the quant methods keep (N-major): the routed
experts' per-channel (format ``fp8``) or 128x128-tile (``fp8_block``)
tensors, and the shared linears' [N, K] weights with per-channel or tile
scales.
"""

import logging

import torch

from qmoe import envs, ops

logger = logging.getLogger(__name__)

FUSED_MOE_DECODE_OP_ATTR = "_fused_moe_decode_op"
_RUNNER_ARMED_ATTR = "_fused_moe_decode_armed"
# the shared expert's tensors, registered on the routed layer
_SHARED_BUFFERS = ("_fmd_w1s", "_fmd_s1s", "_fmd_w2s", "_fmd_s2s", "_fmd_wg")


def fused_moe_decode_supported(quant_method) -> bool:
    """`fused_moe_decode.py:101-102`."""
    return getattr(quant_method, FUSED_MOE_DECODE_OP_ATTR, None) is not None


def _shared_mlp_is_ungated_silu(mlp) -> bool:
    """A shared expert with no gate of its own: gate_up -> silu-and-mul ->
    down (`fused_moe_decode.py:341-350`)."""
    act = getattr(mlp, "act_fn", None)
    act_name = type(act).__name__ if act is not None else ""
    return act_name in ("SiluAndMul", "") and getattr(mlp, "expert_gate", None) is None


def _shared_slice(runner):
    """The shared expert's (w1 [2 I_s, H], w1 scale, w2 [H, I_s], w2 scale,
    gate weight [H] or None), or None when it is not an FP8 MLP the op serves
    (`fused_moe_decode.py:353-407`)."""
    shared = getattr(runner, "_shared_experts", None)
    mlp = getattr(shared, "_layer", shared)
    if mlp is None:
        return None
    gate_up, down = getattr(mlp, "gate_up_proj", None), getattr(mlp, "down_proj", None)
    gate = getattr(mlp, "expert_gate", None)
    if gate_up is None or down is None:
        return None
    if gate is None and not _shared_mlp_is_ungated_silu(mlp):
        return None
    w1, s1 = getattr(gate_up, "weight", None), getattr(gate_up, "weight_scale", None)
    w2, s2 = getattr(down, "weight", None), getattr(down, "weight_scale", None)
    if w1 is None or s1 is None or w2 is None or s2 is None:
        return None
    if w1.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
        return None
    wg = None
    if gate is not None:
        wg = getattr(gate, "weight", None)
        if wg is None or getattr(gate, "bias", None) is not None or wg.numel() != w1.shape[1]:
            return None
    return w1.data, s1.data, w2.data, s2.data, (None if wg is None else wg.data)


def _admit(runner):
    """(shared tensors, routed scale, weight_blocks) for an eligible runner,
    else None (`fused_moe_decode.py:410-474`, one GPU: no mesh conditions)."""
    from qmoe.layers.quantization.fp8 import Fp8MoEMethod

    qm = getattr(runner, "_quant_method", None)
    layer = getattr(runner, "routed_experts", None)
    if not isinstance(qm, Fp8MoEMethod) or layer is None or not getattr(layer, "_qmoe_processed", False):
        return None
    if getattr(layer, "_qmoe_activation", None) != "silu":
        return None
    if getattr(layer, "w13_bias", None) is not None or getattr(layer, "w2_bias", None) is not None:
        return None
    if getattr(runner, "routed_input_transform", None) is not None or \
            getattr(runner, "routed_output_transform", None) is not None:
        return None
    if getattr(runner, "shared_expert_gate", None) is not None:
        return None
    routed_scale = float(getattr(runner, "routed_scaling_factor", 1.0) or 1.0)
    moe = getattr(runner, "moe_config", None) or getattr(layer, "moe_config", None)
    if routed_scale != 1.0 and getattr(moe, "in_dtype", None) == torch.float16:
        return None  # vLLM divides the shared output instead in fp16; not mirrored
    fmt = getattr(layer, "_qmoe_format", None)
    if fmt not in ("fp8", "fp8_block"):
        return None
    shared = _shared_slice(runner)
    if shared is None:
        return None
    w1s, s1s, w2s, s2s, _ = shared
    w1, w2 = layer.w13_weight, layer.w2_weight
    E, N1, H = w1.shape
    I, Is = N1 // 2, w2s.shape[1]
    tiles = fmt == "fp8_block"
    if tiles:
        ok = (tuple(s1s.shape) == (2 * Is // 128, H // 128) and tuple(s2s.shape) == (H // 128, Is // 128))
    else:
        ok = (layer.w13_weight_scale.dim() == 2 and s1s.numel() == 2 * Is and s2s.numel() == H)
    if (not ok or tuple(w2.shape) != (E, H, I) or tuple(w1s.shape) != (2 * Is, H) or tuple(w2s.shape) != (H, Is)
            or I % 128 or Is % 128 or Is > I or H % 512 or H > 16384 or E > 512):
        return None
    return shared, routed_scale, (128 if tiles else None)


def arm_fused_moe_decode(model, what="model") -> int:
    """Arm every eligible MoE runner of `model` (`fused_moe_decode.py:
    513-619`); returns how many were armed. Runners are the modules with a
    ``routed_experts`` layer and a ``_quant_method`` (vLLM's MoERunner)."""
    if not envs.FUSED_MOE_DECODE_KERNEL:
        return 0
    max_tokens = envs.FUSED_MOE_DECODE_KERNEL_MAX_TOKENS
    if max_tokens < 1:
        raise ValueError(f"FUSED_MOE_DECODE_KERNEL_MAX_TOKENS={max_tokens}: must be >= 1.")
    if max_tokens > ops.DECODE_MAX_TOKENS:
        logger.warning("FUSED_MOE_DECODE_KERNEL_MAX_TOKENS=%d: the fused decode op serves at most %d tokens; "
                       "larger steps take the GMM path", max_tokens, ops.DECODE_MAX_TOKENS)
        max_tokens = ops.DECODE_MAX_TOKENS
    # Measured on MI355X (DeepSeek-V3 layer: 256 experts, top 8, 128x128 FP8
    # tiles, shared expert included, graph-replayed): the op matches the GMM
    # path plus the shared linears up to 16 tokens (T = 8 / 16: 386 / 552 vs
    # 385 / 556 us) and is 20-25% slower above (T = 24 / 64: 797 / 1217 vs
    # 647 / 989 us), where its down kernel walks 150-250 experts per column
    # block; larger steps take the GMM path (QMOE_DECODE_OP_MAX_TOKENS)
    max_tokens = max(1, min(max_tokens, envs.QMOE_DECODE_OP_MAX_TOKENS or max_tokens))
    runners = [m for m in model.modules() if hasattr(m, "routed_experts") and hasattr(m, "_quant_method")]
    armed = 0
    for runner in runners:
        admitted = _admit(runner)
        if admitted is None:
            continue
        shared, routed_scale, blocks = admitted
        layer = runner.routed_experts
        for name, tensor in zip(_SHARED_BUFFERS, shared):
            layer.register_buffer(name, tensor, persistent=False)
        setattr(runner._quant_method, FUSED_MOE_DECODE_OP_ATTR,
                dict(max_tokens=max_tokens, routed_scale=routed_scale, weight_blocks=blocks,
                     shared_gated=shared[4] is not None))
        runner._shared_experts = None
        # the op scales the routed experts only; the runner would scale the
        # op's shared + routed sum
        runner.routed_scaling_factor = 1.0
        object.__setattr__(runner, _RUNNER_ARMED_ATTR, True)
        armed += 1
    logger.info("Armed the fused MoE decode op on %d of %d MoE layers of the %s (up to %d tokens; GMM MoE above)",
                armed, len(runners), what, max_tokens)
    return armed


def _shared_expert(x, w1s, s1s, w2s, s2s, wg):
    """The shared MLP as the runner computes it with the op off: FP8 gate_up
    and down linears (the dense quantized matmul), silu-and-mul, and the
    sigmoid gate (`fused_moe_decode.py:144-164`)."""
    from qmoe.layers.linear_common import quantized_matmul

    i_s = w2s.shape[1]
    gu = quantized_matmul(x, w1s.t(), s1s).float()
    mid = (torch.nn.functional.silu(gu[:, :i_s]) * gu[:, i_s:]).to(x.dtype)
    out = quantized_matmul(mid, w2s.t(), s2s).float()
    if wg is not None:
        out = torch.sigmoid(x.float() @ wg.reshape(-1, 1).to(x.dtype).float()) * out
    return out


def fused_moe_decode_routed(quant_method, layer, x, router_logits, input_ids=None):
    """Forward of an armed layer that routes inside the op: the same routes
    as `moe_routing.route` (the layer's plain or grouped rule) and the same
    output as `fused_moe_decode` on them, with the routing folded into the
    op's first launch. None when the step is not served that way (a
    model-supplied routing function, hash routing, non-bf16 hidden states,
    or more tokens than the op takes)."""
    from qmoe.layers import moe_routing

    cfg = getattr(quant_method, FUSED_MOE_DECODE_OP_ATTR)
    if (x.shape[0] > cfg["max_tokens"] or x.dtype != torch.bfloat16
            or getattr(layer, "custom_routing_function", None) is not None
            or (getattr(layer, "hash_indices_table", None) is not None and input_ids is not None)):
        return None
    bias, rsf, ng, tg = moe_routing.routing_params(layer)
    w1s, s1s, w2s, s2s, wg = (getattr(layer, name) for name in _SHARED_BUFFERS)
    out, _, _ = ops.moe_decode_routed(x, router_logits, layer.moe_config.experts_per_token, layer.w13_weight,
                                      layer.w2_weight, layer.w13_weight_scale, layer.w2_weight_scale, w1s, s1s,
                                      w2s, s2s, wg, scoring_func=layer.scoring_func,
                                      renormalize=layer.renormalize, bias=bias, routed_scaling_factor=rsf,
                                      num_expert_group=ng, topk_group=tg, routed_scale=cfg["routed_scale"],
                                      weight_blocks=cfg["weight_blocks"])
    return out


def fused_moe_decode(quant_method, layer, x, topk_weights, topk_ids):
    """Forward of an armed layer: shared + routed experts, bf16 [T, H]
    (`fused_moe_decode.py:622-649`)."""
    cfg = getattr(quant_method, FUSED_MOE_DECODE_OP_ATTR)
    w1s, s1s, w2s, s2s, wg = (getattr(layer, name) for name in _SHARED_BUFFERS)
    T = x.shape[0]
    if T <= cfg["max_tokens"]:
        return ops.moe_decode(x, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale, layer.w2_weight_scale,
                              w1s, s1s, w2s, s2s, wg, topk_weights, topk_ids, routed_scale=cfg["routed_scale"],
                              weight_blocks=cfg["weight_blocks"])
    # above the cap: the GMM MoE, the shared expert and their sum
    from qmoe.layers.fused_moe import fused_moe_gmm

    routed = fused_moe_gmm(x, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale, layer.w2_weight_scale,
                           None, None, topk_weights, topk_ids, None, topk_ids.shape[1], "silu",
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS,
                           weight_format=layer._qmoe_format).float()
    if cfg["routed_scale"] != 1.0:
        routed = routed * cfg["routed_scale"]
    return (routed + _shared_expert(x, w1s, s1s, w2s, s2s, wg)).to(x.dtype)
