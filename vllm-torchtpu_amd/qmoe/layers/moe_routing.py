"""MoE routing (the reference's `moe_routing` / `router_topk` adapters).

``select_experts`` mirrors `layers/adapter/moe_routing.py:232-323`,
``route`` mirrors `:150-186`, and ``rowmax_select`` mirrors
`layers/adapter/router_topk.py:42-50`. Scores, the sort-free top-k (ties to
the lowest expert id), grouped selection, renormalization and scaling all run
in one HIP kernel (`qmoe_moe_route`).
"""

import torch

from qmoe import ops


def rowmax_select(scores: torch.Tensor, topk: int):
    """Top-k of float scores without a sort: (values f32 [R, k], ids int32).

    Scores at or below -3e38 (and NaN) are clamped to -3e38; a row with no
    score above it returns NaN values (`layers/core/rowmax_topk.py:28-61`).
    """
    n = scores.shape[-1]
    if topk > n:
        raise ValueError(f"topk k={topk} exceeds the expert count {n}")
    w, ids = ops.moe_route(scores.float(), topk, scoring_func="none", renormalize=False,
                           weights_f32=True)
    return w.reshape(*scores.shape[:-1], topk), ids.reshape(*scores.shape[:-1], topk)


def select_experts(hidden_states, router_logits, *, topk, renormalize, scoring_fn, layer=None,
                   input_ids=None):
    """(topk_weights in the hidden dtype, topk_ids int32), `moe_routing.py:232-323`.

    Grouped selection (`layer.use_grouped_topk` with ``num_expert_group > 1``
    and ``topk_group < num_expert_group``) uses the DeepSeek-V3 rule that the
    reference delegates to upstream vLLM (`:276-299`).
    """
    if layer is not None and getattr(layer, "hash_indices_table", None) is not None and input_ids is not None:
        raise NotImplementedError("hash routing (DeepSeek-V4) is outside this build's scope")
    bias = getattr(layer, "e_score_correction_bias", None) if layer is not None else None
    rsf = getattr(layer, "routed_scaling_factor", 1.0) if layer is not None else 1.0
    ng, tg = 1, 1
    if (layer is not None and getattr(layer, "use_grouped_topk", False)
            and layer.num_expert_group > 1 and layer.topk_group < layer.num_expert_group):
        ng, tg = layer.num_expert_group, layer.topk_group
    w, ids = ops.moe_route(router_logits, topk, scoring_func=scoring_fn, renormalize=renormalize,
                           bias=bias, routed_scaling_factor=rsf if rsf is not None else 1.0,
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
