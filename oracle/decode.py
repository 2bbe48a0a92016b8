"""The fused decode MoE layer (shared expert + routed experts in one op):
`kernels/experimental/fused_moe_decode/fused_moe_decode_kernel.py:552-740`
(wrapper: route-weight table, active experts, shared gate) and `:200-336`
(kernel body: activation quantization, the two matmuls, the accumulator).

Single device: the all-reduce of the reference (`:395-460`) is the identity
with one rank, and ``expert_start`` is None.

Weights are held N-major here, as the product stores them: ``w1 [E, 2I, H]``
(gate rows then up rows), ``w2 [E, H, I]``; the reference's K-major ``[E, H,
2I]`` / ``[E, I, H]`` copies hold the same values transposed.

The recipe, per token row (all arithmetic float32):

* hidden states: per (row, 512 columns) ``s = max|x| / 448``, ``inv = 0``
  where ``s == 0`` else ``1 / s``, codes ``e4m3(x * inv)`` (`:216-223`);
* first matmul: each 512-column block's dot of codes times that block's row
  scale, summed over blocks; times the per-channel w1 scale (`:286-308`);
* ``mid = silu(gate) * up * coeff`` where ``coeff != 0``, else 0 (`:309-311`),
  ``coeff`` = the bf16-rounded route weight times ``routed_scale`` (summed
  over routes that name the same expert, `:639-646`), or for the shared
  expert ``sigmoid(x . w_g)`` (gated) / 1 (ungated) (`:647-656`);
* ``mid`` quantized like the hidden states, per (row, min(512, I) columns)
  (`:312-319`); second matmul per block, times the block's row scale,
  summed; times the per-channel w2 scale (`:320-330`), added into a float32
  accumulator: the shared expert first, then the active routed experts in
  increasing id order (`:346-393`);
* output: the accumulator rounded to bf16.

``weight_blocks=128`` is this build's variant for checkpoints with 128x128
weight tiles that are kept unrequantized: the
activation blocks are 128 columns, and each block's dot is scaled by the
activation block scale times the weight tile scale before the sum (the
blockwise W8A8 recipe of `tests/kernels/test_quantized_matmul_kernel.py:
66-94`), with no per-channel factor. The reference's kernel only takes
per-channel weights.

Test infrastructure only.
"""

import numpy as np

from oracle.codecs import bf16_round, e4m3_decode, e4m3_encode

QMAX = np.float32(448.0)
DECODE_BLOCK = 512


def quantize_rows_f32(x, block):
    """Per (row, block columns) float32 quantization of `:216-223, 312-319`.
    The last block is partial when the width is not a multiple of the block.
    Returns (uint8 e4m3 codes [M, K], float32 scales [M, ceil(K/block)])."""
    x = np.asarray(x, np.float32)
    m, k = x.shape
    nb = -(-k // block)
    codes = np.zeros((m, k), np.uint8)
    scales = np.zeros((m, nb), np.float32)
    for b in range(nb):
        sl = slice(b * block, min(k, (b + 1) * block))
        blk = x[:, sl]
        s = (np.max(np.abs(blk), axis=1, keepdims=True) / QMAX).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv = np.where(s == 0, np.float32(0.0), (np.float32(1.0) / s)).astype(np.float32)
        codes[:, sl] = e4m3_encode((blk * inv).astype(np.float32))
        scales[:, b] = s[:, 0]
    return codes, scales


def _blocked_dot(xq, xs, wq, block, w_tiles=None):
    """sum_b f32(dot_b(codes)) * xs[:, b] (* w_tiles[n // 128, b]), float32.

    Each block's code dot is exact in float64 and rounded once to float32
    (the reference's f32 MXU result up to its summation order)."""
    m, k = xq.shape
    n = wq.shape[0]
    xv = e4m3_decode(xq).astype(np.float64)
    wv = e4m3_decode(wq).astype(np.float64)
    acc = np.zeros((m, n), np.float32)
    for b in range(-(-k // block)):
        sl = slice(b * block, min(k, (b + 1) * block))
        part = (xv[:, sl] @ wv[:, sl].T).astype(np.float32)
        part = (part * xs[:, b:b + 1]).astype(np.float32)
        if w_tiles is not None:
            part = (part * np.repeat(w_tiles[:, b], 128)[None, :n]).astype(np.float32)
        acc = (acc + part).astype(np.float32)
    return acc


def _silu(v):
    v = np.asarray(v, np.float32)
    return (v * (np.float32(1.0) / (np.float32(1.0) + np.exp(-v.astype(np.float64)).astype(np.float32)))).astype(
        np.float32)


def expert_contribution(xq, xs, coeff, w1q, w1s, w2q, w2s, weight_blocks=None):
    """One expert's term of the accumulator (`accumulate`, `:302-330`) for all
    rows: coeff [M] float32 (0 = the row does not use the expert)."""
    i = w2q.shape[1]
    if weight_blocks is None:
        acc1 = _blocked_dot(xq, xs, w1q, DECODE_BLOCK)
        acc1 = (acc1 * np.asarray(w1s, np.float32)[None, :]).astype(np.float32)
        qb = min(DECODE_BLOCK, i)
    else:
        acc1 = _blocked_dot(xq, xs, w1q, 128, w_tiles=w1s)
        qb = 128
    c = np.asarray(coeff, np.float32)[:, None]
    mid = ((_silu(acc1[:, :i]) * acc1[:, i:]).astype(np.float32) * c).astype(np.float32)
    mid = np.where(c != 0, mid, np.float32(0.0)).astype(np.float32)
    mq, ms = quantize_rows_f32(mid, qb)
    if weight_blocks is None:
        acc2 = _blocked_dot(mq, ms, w2q, qb)
        return (acc2 * np.asarray(w2s, np.float32)[None, :]).astype(np.float32)
    return _blocked_dot(mq, ms, w2q, 128, w_tiles=w2s)


def route_coefficients(topk_weights, topk_ids, num_experts, routed_scale=1.0):
    """`:639-646`: [T, E] float32 coefficients, bf16-rounded weights times
    routed_scale, summed in route order over routes naming the same expert
    (ids outside [0, E) select nothing)."""
    w = bf16_round(np.asarray(topk_weights, np.float32))
    if routed_scale != 1.0:
        w = (w * np.float32(routed_scale)).astype(np.float32)
    ids = np.asarray(topk_ids, np.int64)
    t, k = ids.shape
    coeff = np.zeros((t, num_experts), np.float32)
    for j in range(k):
        sel = ids[:, j:j + 1] == np.arange(num_experts)[None, :]
        coeff = (coeff + sel.astype(np.float32) * w[:, j:j + 1]).astype(np.float32)
    return coeff


def shared_gate_coeff(x, gate_weight):
    """`:647-656`: sigmoid of the f32-accumulated dot of bf16 x with the bf16
    gate weight [H] (None: ungated, coefficient 1)."""
    x = bf16_round(np.asarray(x, np.float32))
    if gate_weight is None:
        return np.ones(x.shape[0], np.float32)
    g = bf16_round(np.asarray(gate_weight, np.float32).reshape(-1)).astype(np.float64)
    d = (x.astype(np.float64) @ g).astype(np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-d.astype(np.float64)).astype(np.float32))).astype(np.float32)


def fused_moe_decode(hidden, w1q, w1s, w2q, w2s, shared_w1q, shared_w1s, shared_w2q, shared_w2s, shared_gate,
                     topk_weights, topk_ids, routed_scale=1.0, weight_blocks=None, return_acc=False):
    """The layer output, bf16-valued float32 [T, H] (the float32 accumulator
    with ``return_acc=True``).

    w1q uint8 e4m3 [E, 2I, H] with w1s [E, 2I] (per channel) or [E, 2I/128,
    H/128] (``weight_blocks=128``); w2q [E, H, I] with w2s [E, H] or [E,
    H/128, I/128]; the shared expert's tensors without the E axis (its
    intermediate size may be smaller). ``shared_gate`` is the gate weight [H]
    or None."""
    x = bf16_round(np.asarray(hidden, np.float32))
    t, h = x.shape
    if h % DECODE_BLOCK:
        raise ValueError(f"hidden size {h} must be a multiple of {DECODE_BLOCK}")
    e_count = w1q.shape[0]
    xb = 128 if weight_blocks else DECODE_BLOCK
    xq, xs = quantize_rows_f32(x, xb)
    coeff = route_coefficients(topk_weights, topk_ids, e_count, routed_scale)
    acc = expert_contribution(xq, xs, shared_gate_coeff(x, shared_gate), shared_w1q, shared_w1s, shared_w2q,
                              shared_w2s, weight_blocks)
    for e in range(e_count):
        if not (coeff[:, e] != 0).any():
            continue
        acc = (acc + expert_contribution(xq, xs, coeff[:, e], w1q[e], w1s[e], w2q[e], w2s[e],
                                         weight_blocks)).astype(np.float32)
    return acc if return_acc else bf16_round(acc)


def decomposed_layer_f32(hidden, w1q, w1s, w2q, w2s, shared_w1q, shared_w1s, shared_w2q, shared_w2s, shared_gate,
                         topk_weights, topk_ids, routed_scale=1.0, skip_expert=None, weight_blocks=None):
    """The reference test's decomposed layer in float (`tests/kernels/
    experimental/test_fused_moe_decode_kernel.py:87-143`): dequantized
    weights, unquantized activations, float64 here; routed_scale scales the
    routed sum only. ``skip_expert`` drops one routed expert (the test's
    positive control)."""
    x = bf16_round(np.asarray(hidden, np.float32)).astype(np.float64)

    def deq(q, s):
        v = e4m3_decode(q).astype(np.float64)
        if weight_blocks is None:
            return v * np.asarray(s, np.float64)[:, None]
        return v * np.repeat(np.repeat(np.asarray(s, np.float64), 128, axis=0), 128, axis=1)[:v.shape[0], :v.shape[1]]

    def ffn(w1, s1, w2, s2):
        gu = x @ deq(w1, s1).T
        i = w2.shape[1]
        g = gu[:, :i]
        return (g / (1.0 + np.exp(-g)) * gu[:, i:]) @ deq(w2, s2).T

    shared = ffn(shared_w1q, shared_w1s, shared_w2q, shared_w2s)
    if shared_gate is not None:
        d = x @ bf16_round(np.asarray(shared_gate, np.float32).reshape(-1)).astype(np.float64)
        shared = shared / (1.0 + np.exp(-d))[:, None]
    tw = bf16_round(np.asarray(topk_weights, np.float32)).astype(np.float64)
    ids = np.asarray(topk_ids, np.int64)
    routed = np.zeros_like(shared)
    for e in range(w1q.shape[0]):
        c = np.where(ids == e, tw, 0.0).sum(axis=1, keepdims=True)
        if e == skip_expert or not (c != 0).any():
            continue
        routed += c * ffn(w1q[e], w1s[e], w2q[e], w2s[e])
    return routed_scale * routed + shared
