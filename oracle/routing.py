"""MoE routing references. Test infrastructure only.

Scores are evaluated in float64 and rounded once to float32 (the correctly
rounded float32 score). The reference evaluates them with float32 library
routines (`adapter/moe_routing.py:189-201`), which may differ from this by one
ulp; the build's GPU router uses the same float64-then-round definition so
that expert ids -- which depend on exact score comparisons once a bias is
added -- are reproducible bit for bit on both sides. For softmax without a
bias the ids do not depend on the last bit at all (softmax is monotonic in the
logit, and distinct bf16 logits differ by far more than an ulp of the score).
"""

import numpy as np

from oracle.codecs import bf16_round

NEG = np.float32(-3.0e38)  # `layers/core/rowmax_topk.py:26`


def scores_of(logits, scoring_func):
    """`moe_routing.py:189-201` (`_apply_scoring_fn`) on float32 logits."""
    x = np.asarray(logits, np.float32).astype(np.float64)
    if scoring_func == "softmax":
        mx = np.max(x, axis=-1, keepdims=True)
        e = np.exp(x - mx)
        s = e / np.sum(e, axis=-1, keepdims=True)
    elif scoring_func == "sigmoid":
        s = 1.0 / (1.0 + np.exp(-x))
    elif scoring_func == "sqrtsoftplus":
        s = np.sqrt(np.logaddexp(0.0, x))
    else:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    return s.astype(np.float32)


def rowmax_topk(scores, k):
    """`layers/core/rowmax_topk.py:28-61`: k passes of (row max -> lowest
    column attaining it -> mask it). Scores <= NEG (and NaN) are clamped to
    NEG; a row whose best score is <= NEG gets NaN weights. Returns
    (values f32 [R, k], ids int32 [R, k])."""
    s = np.asarray(scores, np.float32)
    n = s.shape[-1]
    if k > n:
        raise ValueError(f"topk k={k} exceeds the expert count {n}")
    masked = np.finfo(np.float32).min
    cur = np.where(s > NEG, s, NEG).astype(np.float32)
    iota = np.arange(n, dtype=np.int32)
    vals, ids = [], []
    for _ in range(k):
        m = np.max(cur, axis=-1, keepdims=True)
        idx = np.min(np.where(cur == m, iota, n - 1), axis=-1, keepdims=True)
        vals.append(m)
        ids.append(idx)
        cur = np.where(iota == idx, masked, cur).astype(np.float32)
    w = np.concatenate(vals, axis=-1).astype(np.float32)
    i = np.concatenate(ids, axis=-1).astype(np.int32)
    w = np.where(w[..., :1] <= NEG, np.float32("nan"), w).astype(np.float32)
    return w, i


def _finish(w, renormalize, routed_scaling_factor):
    """`moe_routing.py:315-323`: renormalize with a 1e-20 clamp, scale, bf16."""
    w = np.asarray(w, np.float32)
    if renormalize:
        w = (w / np.maximum(np.sum(w, axis=-1, keepdims=True, dtype=np.float32),
                            np.float32(1e-20))).astype(np.float32)
    if routed_scaling_factor != 1.0:
        w = (w * np.float32(routed_scaling_factor)).astype(np.float32)
    return bf16_round(w)


def select_experts(logits, topk, renormalize, scoring_func="softmax",
                   e_score_correction_bias=None, routed_scaling_factor=1.0):
    """`moe_routing.py:232-323` (`select_experts`, non-grouped branch).

    With a bias, experts are CHOSEN by ``scores + bias`` (float32 add) and
    WEIGHTED by the unbiased scores (`:306-311`). Returns (weights as bf16
    values in f32 [T, k], ids int32 [T, k])."""
    s = scores_of(logits, scoring_func)
    if e_score_correction_bias is not None:
        choice = (s + np.asarray(e_score_correction_bias, np.float32)[None, :]).astype(np.float32)
        _, ids = rowmax_topk(choice, topk)
        w = np.take_along_axis(s, ids.astype(np.int64), axis=-1)
    else:
        w, ids = rowmax_topk(s, topk)
    return _finish(w, renormalize, routed_scaling_factor), ids


def grouped_topk(logits, topk, renormalize, num_expert_group, topk_group,
                 scoring_func="sigmoid", e_score_correction_bias=None,
                 routed_scaling_factor=1.0):
    """Grouped (DeepSeek-V3) routing, the build's definition.

    parity unpinned: the reference delegates to upstream vLLM v0.32.0
    ``grouped_topk`` (call site `adapter/moe_routing.py:276-299`), which is not
    vendored, and its own tests mock it. Restated from the DeepSeek-V3 method:

    1. ``s = score(logits)``; ``c = s + bias`` (or ``s`` without a bias);
    2. group score = sum of the two largest ``c`` in the group (max without a
       bias);
    3. keep the ``topk_group`` best groups (rowmax order, ties -> lowest group);
    4. choose ``topk`` experts from the kept groups by ``c`` (rowmax order,
       ties -> lowest id; the returned order is descending ``c``);
    5. weights = unbiased ``s`` at the chosen ids; renormalize; scale; bf16.
    """
    s = scores_of(logits, scoring_func)
    t, e = s.shape
    g = num_expert_group
    if e_score_correction_bias is not None:
        c = (s + np.asarray(e_score_correction_bias, np.float32)[None, :]).astype(np.float32)
        cg = c.reshape(t, g, e // g)
        two, _ = rowmax_topk(cg.reshape(t * g, e // g), 2)
        gs = (two[:, 0] + two[:, 1]).astype(np.float32).reshape(t, g)
    else:
        c = s
        gs = np.max(c.reshape(t, g, e // g), axis=-1)
    _, gids = rowmax_topk(gs, topk_group)
    keep = np.zeros((t, g), bool)
    np.put_along_axis(keep, gids.astype(np.int64), True, axis=-1)
    mask = np.repeat(keep, e // g, axis=-1)
    cm = np.where(mask, c, np.float32(-np.inf)).astype(np.float32)
    # every kept score is > NEG for finite inputs, so the sentinel clamp of
    # rowmax_topk never selects a masked expert when topk <= kept experts.
    _, ids = rowmax_topk(cm, topk)
    w = np.take_along_axis(s, ids.astype(np.int64), axis=-1)
    return _finish(w, renormalize, routed_scaling_factor), ids


def hash_select(logits, hash_indices_table, input_ids, renormalize, scoring_func="softmax",
                routed_scaling_factor=1.0):
    """`moe_routing.py:204-229` (`_hash_moe_select`, DeepSeek-V4 hash
    routing, taken by `select_experts` when the layer has a
    `hash_indices_table` and input ids are given, `:259-274`): expert ids are
    ``table[input_ids]`` and the weights the row's (unbiased) scores at those
    ids, renormalized and scaled like every other branch."""
    s = scores_of(logits, scoring_func)
    ids = np.asarray(hash_indices_table, np.int64)[np.asarray(input_ids, np.int64).reshape(-1)]
    w = np.take_along_axis(s, ids, axis=-1)
    return _finish(w, renormalize, routed_scaling_factor), ids.astype(np.int32)
