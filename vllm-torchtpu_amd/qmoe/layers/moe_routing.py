"""MoE routing (the reference's `moe_routing` / `router_topk` adapters).

``select_experts`` mirrors `layers/adapter/moe_routing.py:232-323`,
``route`` mirrors `:150-186`, and ``rowmax_select`` mirrors
`layers/adapter/router_topk.py:42-50`. Scores, the sort-free top-k (ties to
the lowest expert id), grouped selection, renormalization and scaling all run
in one HIP kernel (`qmoe_moe_route`), registered as the torch custom op
``torch.ops.qmoe.moe_route`` with a fake implementation (the reference
registers its router op the same way, `layers/adapter/router_topk.py:36-39`).
"""

from typing import Optional, Tuple

import torch

from qmoe import ops


@torch.library.custom_op("qmoe::moe_route", mutates_args=())
def _moe_route_op(logits: torch.Tensor, topk: int, scoring_func: str, renormalize: bool,
                  bias: Optional[torch.Tensor], routed_scaling_factor: float, num_expert_group: int,
                  topk_group: int, weights_f32: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    return ops.moe_route(logits, topk, scoring_func, renormalize, bias, routed_scaling_factor,
                         num_expert_group, topk_group, weights_f32)


@_moe_route_op.register_fake
def _(logits, topk, scoring_func, renormalize, bias, routed_scaling_factor, num_expert_group, topk_group,
      weights_f32):
    T = logits.numel() // logits.shape[-1]
    w = logits.new_empty((T, topk), dtype=torch.float32 if weights_f32 else torch.bfloat16)
    return w, logits.new_empty((T, topk), dtype=torch.int32)


@torch.library.custom_op("qmoe::moe_route_hash", mutates_args=())
def _moe_route_hash_op(logits: torch.Tensor, topk: int, table: torch.Tensor, input_ids: torch.Tensor,
                       scoring_func: str, renormalize: bool,
                       routed_scaling_factor: float) -> Tuple[torch.Tensor, torch.Tensor]:
    return ops.moe_route_hash(logits, topk, table, input_ids, scoring_func, renormalize, routed_scaling_factor)


@_moe_route_hash_op.register_fake
def _(logits, topk, table, input_ids, scoring_func, renormalize, routed_scaling_factor):
    T = logits.numel() // logits.shape[-1]
    return (logits.new_empty((T, topk), dtype=torch.bfloat16), logits.new_empty((T, topk), dtype=torch.int32))


def _route(logits, topk, scoring_func, renormalize, bias=None, routed_scaling_factor=1.0,
           num_expert_group=1, topk_group=1, weights_f32=False):
    """Host-side checks (raised at trace time), then the custom op."""
    if scoring_func not in ops._SCORING:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    if topk > logits.shape[-1]:
        raise ValueError(f"topk k={topk} exceeds the expert count {logits.shape[-1]}")
    return torch.ops.qmoe.moe_route(logits, int(topk), scoring_func, bool(renormalize), bias,
                                    float(routed_scaling_factor), int(num_expert_group or 1),
                                    int(topk_group or 1), bool(weights_f32))


def rowmax_select(scores: torch.Tensor, topk: int):
    """Top-k of float scores without a sort: (values f32 [R, k], ids int32).

    Scores at or below -3e38 (and NaN) are clamped to -3e38; a row with no
    score above it returns NaN values (`layers/core/rowmax_topk.py:28-61`).
    """
    n = scores.shape[-1]
    if topk > n:
        raise ValueError(f"topk k={topk} exceeds the expert count {n}")
    w, ids = _route(scores.float(), topk, "none", False, weights_f32=True)
    return w.reshape(*scores.shape[:-1], topk), ids.reshape(*scores.shape[:-1], topk)


def routing_params(layer):
    """The layer's routing settings as `select_experts` reads them: (bias,
    routed_scaling_factor, num_expert_group, topk_group); grouped selection
    only when `use_grouped_topk` with num_expert_group > 1 and topk_group <
    num_expert_group (`moe_routing.py:276-299`)."""
    bias = getattr(layer, "e_score_correction_bias", None) if layer is not None else None
    rsf = getattr(layer, "routed_scaling_factor", 1.0) if layer is not None else 1.0
    ng, tg = 1, 1
    if (layer is not None and getattr(layer, "use_grouped_topk", False)
            and layer.num_expert_group > 1 and layer.topk_group < layer.num_expert_group):
        ng, tg = layer.num_expert_group, layer.topk_group
    return bias, (rsf if rsf is not None else 1.0), ng, tg


def select_experts(hidden_states, router_logits, *, topk, renormalize, scoring_fn, layer=None,
                   input_ids=None):
    """(topk_weights in the hidden dtype, topk_ids int32), `moe_routing.py:232-323`.

    Grouped selection (`layer.use_grouped_topk` with ``num_expert_group > 1``
    and ``topk_group < num_expert_group``) uses the DeepSeek-V3 rule that the
    reference delegates to upstream vLLM (`:276-299`).
    """
    table = getattr(layer, "hash_indices_table", None) if layer is not None else None
    if table is not None and input_ids is not None:
        # DeepSeek-V4 hash routing (`moe_routing.py:259-274`): ids from the
        # table row of each token's input id, weights from its scores
        rsf = getattr(layer, "routed_scaling_factor", 1.0)
        if scoring_fn not in ops._SCORING:
            raise NotImplementedError(f"FusedMoE does not support {scoring_fn} scoring function for TPU.")
        w, ids = torch.ops.qmoe.moe_route_hash(router_logits, int(topk), table, input_ids, scoring_fn,
                                               bool(renormalize), float(rsf if rsf is not None else 1.0))
        return w.to(hidden_states.dtype), ids
    bias, rsf, ng, tg = routing_params(layer)
    w, ids = _route(router_logits, topk, scoring_fn, renormalize, bias=bias, routed_scaling_factor=rsf,
                    num_expert_group=ng, topk_group=tg)
    return w.to(hidden_states.dtype), ids


def route(layer, hidden_states, router_logits, input_ids=None):
    """Routing entry of the MoE methods, `moe_routing.py:150-186`: a
    model-supplied ``custom_routing_function`` wins, else `select_experts`."""
    topk = layer.moe_config.experts_per_token
    custom = getattr(layer, "custom_routing_function", None)
    if custom is not None:
        return custom(hidden_states=hidden_states, gating_output=router_logits, topk=topk,
                      renormalize=layer.renormalize)
    return select_experts(hidden_states, router_logits, topk=topk, renormalize=layer.renormalize,
                          scoring_fn=layer.scoring_func, layer=layer, input_ids=input_ids)
