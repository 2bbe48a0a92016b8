"""Fused-MoE references: permutation metadata, activations, full layer.

Test infrastructure only.
"""

import numpy as np

from oracle.codecs import bf16_round, dequant_int4, dequant_mxfp4, dequant_nvfp4, e4m3_decode, e5m2_decode
from oracle.linear import _mm, w8a8_gmm, w8a8_gmm_bf16acc
from oracle.quant import quantize_act, quantize_mx_fp4


def prepare_routed(topk_ids, topk_weights=None, num_experts=None, skip_padded_tokens=False):
    """`layers/core/fused_moe_gmm.py:288-408` (`prepare_routed_gmm_inputs`,
    non-EP, non-SparseCore branch).

    Flattens ``[T, k]`` ids to ``T*k`` routes; a route is valid when its id is
    >= 0 (and, with ``skip_padded_tokens``, its weight is non-zero,
    `:314-320`); invalid routes sort after every expert (key ``E``). The sort
    is a STABLE argsort of the keys (`:337-378`; the single packed sort of
    `:272-285` orders equal keys by flat position, which is the same thing).

    Returns dict(sorted_idx, revert, group_sizes, token_sorted, valid).
    """
    ids = np.asarray(topk_ids, np.int64)
    t, k = ids.shape
    flat = ids.reshape(-1)
    valid = flat >= 0
    if skip_padded_tokens:
        valid &= np.asarray(topk_weights, np.float32).reshape(-1) != 0
    keys = np.where(valid, flat, num_experts)
    sorted_idx = np.argsort(keys, kind="stable").astype(np.int32)
    revert = np.argsort(sorted_idx, kind="stable").astype(np.int32)
    group_sizes = np.bincount(flat[valid], minlength=num_experts).astype(np.int32)
    return dict(
        sorted_idx=sorted_idx,
        revert=revert,
        group_sizes=group_sizes,
        token_sorted=(sorted_idx // k).astype(np.int32),
        valid=valid,
    )


def _sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def _gelu_tanh(x):
    x = x.astype(np.float64)
    return (0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))).astype(np.float32)


def act_fn(gate, up, activation):
    """`kernels/megablox/gmm_v2.py:30-58, 84-122` (`apply_act_fn`).

    ``gelu`` is jax.nn.gelu with its default ``approximate=True``, i.e. the
    same tanh form as ``gelu_tanh``.
    """
    g = np.asarray(gate, np.float32)
    u = np.asarray(up, np.float32)
    if activation == "silu":
        return g * _sigmoid(g) * u
    if activation in ("gelu", "gelu_tanh"):
        return _gelu_tanh(g) * u
    if activation == "swigluoai":
        g = np.minimum(g, np.float32(7.0))
        u = np.clip(u, np.float32(-7.0), np.float32(7.0))
        return (u + np.float32(1.0)) * (g * _sigmoid(np.float32(1.702) * g))
    if activation == "silu_and_mul_with_clamp":
        g = np.minimum(g, np.float32(10.0))
        u = np.clip(u, np.float32(-10.0), np.float32(10.0))
        return g * _sigmoid(g) * u
    if activation.startswith("situ:"):
        _, beta, lin = activation.split(":")
        beta = float(beta)
        gg = (beta * np.tanh(g.astype(np.float64) / beta) * _sigmoid(g)).astype(np.float32)
        if lin != "none":
            lb = float(lin)
            u = (lb * np.tanh(u.astype(np.float64) / lb)).astype(np.float32)
        return gg * u
    raise NotImplementedError(f"Unsupported activation function: {activation}")


class ExpertWeights:
    """Dequantized view of one expert format, for the reference loops.

    fmt:
      "mxfp4": w13 packed u8 [E, 2I, H/2] + e8m0 [E, 2I, H/32]; w2 [E, H, I/2] + [E, H, I/32]
      "nvfp4": w13 packed u8 [E, 2I, H/2] + f32 fused scales [E, 2I, H/16]; w2 likewise
      "int4": w13 int32 carriers [E, 2I, H/8] + bf16-valued scales [E, 2I, H/group]; w2 likewise
      "fp8_block": w13 e4m3 [E, 2I, H] + tile scale_inv [E, 2I/128, H/128]; w2 likewise
      "fp8" / "int8": w13 e4m3 / int8 [E, 2I, H] + per-channel scale [E, 2I] (or per (row, B
          columns) [E, 2I, H/B]); w2 [E, H, I] + [E, H]
      "fp8_bf16acc": as "fp8" (per-channel), each expert linear with the grouped matmul's own
          bf16 accumulator (``linear.w8a8_gmm_bf16acc``, `gmm_v2.py:508-560` as written) and
          silu applied in bf16 (``silu_mul_bf16``)
      "fp8_w8a16": w13 e4m3 [E, 2I, H] + per-(row, 128) scale [E, 2I, H/128]; w2 likewise
      "fp8_rowquant" / "int8_rowquant": as "fp8" / "int8" with per-channel scales
      "bf16": w13 [E, 2I, H] f32 (bf16 values); w2 [E, H, I]
      "mxfp4_mx": weights as "mxfp4" (unpadded); each expert linear's input rows (the
          gathered tokens, the bf16 intermediate) MX-quantized per 32 columns
          (``quant.quantize_mx_fp4``) and dequantized exactly: the opt-in W4A4 regime
    Activations: bf16 for mxfp4/nvfp4/int4/bf16 (W4A16 / W16A16) and fp8_w8a16 (weights
    dequantized to bf16(code * bf16(scale)), `kernels/megablox/gmm_v2.py:452-462`);
    per-(row, 128) e4m3 for fp8_block (the blockwise W8A8 recipe of config 4); per-(row,
    512) bf16-arithmetic codes for fp8 / int8 (the grouped matmul's quantized-lhs regime,
    `gmm_v2.py:500-548`, restated in ``linear.w8a8_gmm``); per-row codes for the
    rowquant formats (`kernels/quantized_matmul/util.py:80-124`).
    """

    def __init__(self, fmt, w13, w13_scale, w2, w2_scale, b13=None, b2=None, keep=True):
        self.fmt, self.w13, self.s13, self.w2, self.s2 = fmt, w13, w13_scale, w2, w2_scale
        self.b13, self.b2 = b13, b2
        self.keep = keep  # keep dequantized experts (False: bounded memory for large expert sets)
        self._cache = {}

    def dense(self, which, e):
        key = (which, e)
        if not self.keep:
            self._cache.clear()
        if key not in self._cache:
            w = self.w13[e] if which == 13 else self.w2[e]
            s = None
            if self.fmt != "bf16":
                s = self.s13[e] if which == 13 else self.s2[e]
            if self.fmt in ("mxfp4", "mxfp4_mx"):
                d = dequant_mxfp4(w, s)
            elif self.fmt == "nvfp4":
                d = dequant_nvfp4(w, s)
            elif self.fmt == "int4":
                d = dequant_int4(w, s)
            elif self.fmt in ("fp8_block", "fp8", "fp8_bf16acc", "fp8_w8a16", "fp8_rowquant"):
                d = e4m3_decode(w)
            elif self.fmt == "e5m2":
                d = e5m2_decode(w)
            elif self.fmt in ("int8", "int8_rowquant"):
                d = np.asarray(w, np.int8).astype(np.float32)
            else:
                d = np.asarray(w, np.float32)
            self._cache[key] = d
        return self._cache[key]

    def linear(self, which, e, x):
        """x bf16-valued [R, K] -> f32 [R, N] for expert e."""
        s = None if self.fmt == "bf16" else (self.s13[e] if which == 13 else self.s2[e])
        if self.fmt in ("fp8", "int8", "e5m2"):
            w = self.w13[e] if which == 13 else self.w2[e]
            qd = "fp8" if self.fmt == "e5m2" else self.fmt  # float weights meet e4m3 activations
            out, _, _ = w8a8_gmm(x, w, s, qd, round_out=False, wdtype=self.fmt)
        elif self.fmt == "fp8_bf16acc":
            w = self.w13[e] if which == 13 else self.w2[e]
            out = w8a8_gmm_bf16acc(x, w, s, "fp8")
        elif self.fmt == "fp8_w8a16":
            wv = self.dense(which, e)
            sb = np.repeat(bf16_round(np.asarray(s, np.float32)), 128, axis=1)[:, :wv.shape[1]]
            out = _mm(x, bf16_round((wv * sb).astype(np.float32)))
        elif self.fmt in ("fp8_rowquant", "int8_rowquant"):
            qd = self.fmt.split("_")[0]
            xq, xs = quantize_act(x, qd)
            xv = e4m3_decode(xq) if qd == "fp8" else xq.astype(np.float32)
            wv = self.dense(which, e)
            out = (_mm(xv, wv) * xs[:, None]).astype(np.float32) if qd == "fp8" else \
                (np.matmul(xq.astype(np.float64), wv.astype(np.float64).T).astype(np.float32) * xs[:, None]).astype(np.float32)
            out = (out * np.asarray(s, np.float32)[None, :]).astype(np.float32)
        elif self.fmt == "mxfp4_mx":
            xq, xs = quantize_mx_fp4(x)
            out = _mm(dequant_mxfp4(xq, xs), self.dense(which, e))
        elif self.fmt != "fp8_block":
            out = _mm(x, self.dense(which, e))
        else:
            wv = self.dense(which, e)
            n, k = wv.shape
            xq, xs = quantize_act(x, "fp8", block=128)
            xv = e4m3_decode(xq)
            out = np.zeros((x.shape[0], n), np.float32)
            sb = np.repeat(s, 128, axis=0)[:n]  # [N, K/128]
            for b in range(k // 128):
                sl = slice(b * 128, (b + 1) * 128)
                d = _mm(xv[:, sl], wv[:, sl])
                out += (d * xs[:, b:b + 1]).astype(np.float32) * sb[None, :, b]
        bias = self.b13 if which == 13 else self.b2
        if bias is not None:
            out = out + np.asarray(bias[e], np.float32)[None, :]
        return out.astype(np.float32)


def fused_moe(hidden, weights: ExpertWeights, topk_weights, topk_ids, activation,
              skip_padded_tokens=False):
    """Grouped form of `layers/core/fused_moe_gmm.py:592-728` (non-EP):

    permute by expert (`prepare_routed`), gmm1 with the fused activation and a
    bf16 result (gmm_v2's output dtype is the lhs dtype, `:441-453`), gmm2,
    then the weighted unpermute ``sum_k w[t,k] * y[revert[t*k+k']]`` over valid
    routes (`:572-577`). Accumulation is kept in float32 up to the final bf16
    cast; the reference's intermediate bf16 roundings after gmm2 are within
    the tolerance the parity tests state.

    Also returns the intermediate (post-activation, bf16) rows in sorted order
    for kernel-level checks.
    """
    x = np.asarray(hidden, np.float32)
    t, h = x.shape
    ids = np.asarray(topk_ids)
    k = ids.shape[1]
    num_experts = weights.w13.shape[0]
    meta = prepare_routed(ids, topk_weights, num_experts, skip_padded_tokens)
    w = bf16_round(np.asarray(topk_weights, np.float32))  # `:653` weights -> bf16
    gs = meta["group_sizes"]
    offs = np.concatenate([[0], np.cumsum(gs)])
    n_valid = int(offs[-1])
    inter_rows = None
    y_sorted = np.zeros((t * k, h), np.float32)
    for e in range(num_experts):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if lo == hi:
            continue
        rows = x[meta["token_sorted"][lo:hi]]
        gu = weights.linear(13, e, rows)
        i = gu.shape[1] // 2
        if weights.fmt == "fp8_bf16acc" and activation == "silu":
            a = silu_mul_bf16(gu[:, :i], gu[:, i:])
        else:
            a = bf16_round(act_fn(gu[:, :i], gu[:, i:], activation))
        if inter_rows is None:
            inter_rows = np.zeros((t * k, i), np.float32)
        inter_rows[lo:hi] = a
        y_sorted[lo:hi] = weights.linear(2, e, a)
    out = np.zeros((t, h), np.float32)
    flat_w = w.reshape(-1)
    for r in range(t * k):
        pos = meta["revert"][r]
        if pos < n_valid and meta["valid"][r]:
            out[r // k] += flat_w[r] * y_sorted[pos]
    return bf16_round(out), meta, inter_rows


def fused_moe_tokens(hidden_rows, weights: ExpertWeights, topk_weights, topk_ids, activation,
                     num_experts, skip_padded_tokens=False):
    """The layer for a subset of tokens, one token at a time: the per-token
    loop of the reference's test oracle `_reference_fused_moe`
    (`tests/layers/core/test_fused_moe_gmm.py:387-427`: for each valid slot,
    gate_up, activation, down, times the routing weight, summed over slots
    in f32), with the arithmetic of `fused_moe` above (per-format expert
    linears, bf16 intermediate, bf16 routing weights, ids outside
    [0, num_experts) skipped as the permutation does). Every quantity of a
    token depends on that token's row only, so the rows equal `fused_moe`'s
    rows for the same tokens; this form touches only the experts the given
    tokens route to.

    hidden_rows [R, H], topk_weights / topk_ids [R, k] -> bf16-valued f32 [R, H].
    """
    x = np.asarray(hidden_rows, np.float32)
    ids = np.asarray(topk_ids)
    w = bf16_round(np.asarray(topk_weights, np.float32))
    r, h = x.shape
    out = np.zeros((r, h), np.float32)
    for t in range(r):
        acc = np.zeros(h, np.float32)
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            if e < 0 or e >= num_experts or (skip_padded_tokens and w[t, j] == 0):
                continue
            gu = weights.linear(13, e, x[t:t + 1])
            i = gu.shape[1] // 2
            a = bf16_round(act_fn(gu[:, :i], gu[:, i:], activation))
            acc += w[t, j] * weights.linear(2, e, a)[0]
        out[t] = acc
    return bf16_round(out)


def silu_mul_bf16(g, u):
    """``jax.nn.silu(g) * u`` on bf16 arrays, as the grouped matmul applies it
    to its bf16 accumulator (`kernels/megablox/gmm_v2.py:575`) and the
    dense-expert kernel to its own (`moe_dense_expert.py:152`): ``sigmoid``,
    ``g * sigmoid`` and ``* u`` each rounded to bf16."""
    g = bf16_round(np.asarray(g, np.float32))
    return bf16_round(bf16_round(g * bf16_round(_sigmoid(g))) * bf16_round(np.asarray(u, np.float32)))


def dense_expert_moe(hidden, w13, s13, w2, s2, topk_weights, topk_ids):
    """The dense-expert decode branch, `kernels/experimental/moe_dense_expert.py:
    112-190, 249-270` (taken by `layers/core/fused_moe_gmm.py:669-686`), in
    this package's expert layout: w13 e4m3 codes [E, 2I, H] ([gate | up]
    rows), w2 [E, H, I], per-channel f32 scales s13 [E, 2I], s2 [E, H].

    * Routing coefficients ``coeff[t, e] = sum over routes of f32(bf16(w))``
      for the routes of token t to expert e (repeated ids merge; ids outside
      [0, E) add nothing), `:256-262`; an expert is active when any of its
      coefficients is non-zero.
    * Per active expert, ascending id: gate_up as the grouped matmul's
      quantized-lhs regime with its bf16 accumulator (`:131-151`:
      per (row, 512) e4m3 codes with bf16 scales, bf16 block dot, times the
      activation scale, times bf16(weight scale), bf16 sums; this is
      ``linear.w8a8_gmm_bf16acc``); ``silu(gate) * up`` with jax's bf16
      elementwise rounding (``sigmoid``, ``gate * sigmoid``, ``* up`` each
      rounded to bf16, `:152`); the same recipe for down (`:153-168`).
    * ``owner[t] += coeff[t, e] * f32(down)`` where ``coeff != 0``, else 0
      (the mask keeps a non-finite expert output out of tokens that do not
      route to it, `:169-172`); the result is bf16(owner) (`:246`).

    Every token's rows depend on that token only, so the expert linears run
    on the tokens with a non-zero coefficient; the others are masked anyway.

    hidden [T, H] bf16-valued; topk_weights / topk_ids [T, k] -> [T, H]
    bf16-valued f32.
    """
    x = bf16_round(np.asarray(hidden, np.float32))
    t, h = x.shape
    ids = np.asarray(topk_ids)
    w = bf16_round(np.asarray(topk_weights, np.float32))
    num_experts = np.asarray(w13).shape[0]
    coeff = np.zeros((t, num_experts), np.float32)
    for r in range(ids.shape[1]):
        for tok in range(t):
            e = int(ids[tok, r])
            if 0 <= e < num_experts:
                coeff[tok, e] = np.float32(coeff[tok, e] + w[tok, r])
    owner = np.zeros((t, h), np.float32)
    for e in range(num_experts):
        rows = np.nonzero(coeff[:, e] != 0)[0]
        if rows.size == 0:
            continue
        gu = w8a8_gmm_bf16acc(x[rows], w13[e], s13[e], "fp8")
        i = gu.shape[1] // 2
        a = silu_mul_bf16(gu[:, :i], gu[:, i:])
        y = w8a8_gmm_bf16acc(a, w2[e], s2[e], "fp8")
        owner[rows] = (owner[rows] + (y * coeff[rows, e][:, None]).astype(np.float32)).astype(np.float32)
    return bf16_round(owner)

