"""Pins the MoE oracle (`oracle/moe.py`): permutation metadata against the
reference's known answer and its single-sort procedure, activations against
closed forms, and the grouped layer against a per-token loop. CPU only."""

import numpy as np
import pytest

from oracle import codecs, moe


def test_prepare_routed_known_answer():
    """`tests/layers/core/test_fused_moe_gmm.py:430-467`, answers written out:
    ids [[1,0],[0,-1],[1,0]] -> keys [1,0,0,2,1,0]."""
    meta = moe.prepare_routed(np.array([[1, 0], [0, -1], [1, 0]]), num_experts=2)
    assert meta["sorted_idx"].tolist() == [1, 2, 5, 0, 4, 3]
    assert meta["revert"].tolist() == [3, 0, 1, 5, 4, 2]
    assert meta["token_sorted"].tolist() == [0, 1, 2, 0, 2, 1]
    assert meta["group_sizes"].tolist() == [3, 2]
    assert meta["valid"].tolist() == [True, True, True, False, True, True]


def _single_sort(keys, k):
    """`layers/core/fused_moe_gmm.py:272-285`: one sort of the packed unique
    integers key << flat_bits | flat position (any sort order of unique keys
    is the same), unpacked into (sorted_idx, revert, token_sorted)."""
    n = keys.shape[0]
    bits = max(1, (n - 1).bit_length())
    packed = np.sort((keys.astype(np.int64) << bits) | np.arange(n))
    sorted_idx = packed & ((1 << bits) - 1)
    revert = np.empty(n, np.int64)
    revert[sorted_idx] = np.arange(n)
    return sorted_idx, revert, sorted_idx // k


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (4, 10, 64), (204, 10, 64), (16, 1, 8), (33, 4, 128)])
def test_prepare_routed_matches_packed_single_sort(T, k, E):
    """Invariants of `tests/layers/adapter/test_moe_single_sort.py:35-119`:
    the stable argsort and the packed single sort agree (incl. invalid
    routes, all-equal keys and k = 1)."""
    rng = np.random.default_rng(T * 100 + k)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[rng.random(ids.shape) < 0.1] = -1
    meta = moe.prepare_routed(ids, num_experts=E)
    keys = np.where(ids.reshape(-1) >= 0, ids.reshape(-1), E)
    si, rv, ts = _single_sort(keys, k)
    np.testing.assert_array_equal(meta["sorted_idx"], si)
    np.testing.assert_array_equal(meta["revert"], rv)
    np.testing.assert_array_equal(meta["token_sorted"], ts)
    np.testing.assert_array_equal(meta["group_sizes"], np.bincount(keys, minlength=E + 1)[:E])


def test_all_equal_keys_keep_flat_order():
    meta = moe.prepare_routed(np.zeros((16, 1), np.int32), num_experts=4)
    assert meta["sorted_idx"].tolist() == list(range(16))


def test_skip_padded_routes_sort_last():
    """`fused_moe_gmm.py:314-320`: a zero routing weight makes a route
    invalid when skip_padded_tokens is set."""
    ids = np.array([[0, 1], [1, 0]], np.int32)
    w = np.array([[0.5, 0.0], [0.25, 0.75]], np.float32)
    meta = moe.prepare_routed(ids, w, 2, skip_padded_tokens=True)
    assert meta["group_sizes"].tolist() == [2, 1]
    assert meta["sorted_idx"].tolist() == [0, 3, 2, 1]


def test_swigluoai_closed_form():
    """`gmm_v2.py:30-38`: g = min(g, 7), u = clip(u, -7, 7),
    (u + 1) * g * sigmoid(1.702 g)."""
    g = np.array([8.0, -2.0, 0.5], np.float32)
    u = np.array([-9.0, 9.0, 0.25], np.float32)
    got = moe.act_fn(g, u, "swigluoai")
    sig = lambda x: 1 / (1 + np.exp(-x))  # noqa: E731
    want = [(-7 + 1) * 7 * sig(1.702 * 7), (7 + 1) * -2 * sig(-3.404), 1.25 * 0.5 * sig(0.851)]
    np.testing.assert_allclose(got, want, rtol=1e-6)


@pytest.mark.parametrize("linear_beta", ["none", "25.0"])
def test_situ_known_form(linear_beta):
    """`tests/kernels/test_gmm_v2.py:57-68`."""
    g = np.array([-3.0, 0.5, 7.0], np.float32)
    u = np.array([-30.0, 2.0, 40.0], np.float32)
    eg = 4.0 * np.tanh(g / 4.0) / (1 + np.exp(-g))
    eu = u if linear_beta == "none" else 25.0 * np.tanh(u / 25.0)
    np.testing.assert_allclose(moe.act_fn(g, u, f"situ:4.0:{linear_beta}"), eg * eu, rtol=1e-5, atol=1e-5)


def test_silu_and_clamp_and_gelu_points():
    g = np.array([0.0, 12.0, -1.0], np.float32)
    u = np.array([3.0, -20.0, 2.0], np.float32)
    sig = lambda x: 1 / (1 + np.exp(-x))  # noqa: E731
    np.testing.assert_allclose(moe.act_fn(g, u, "silu"), g * sig(g) * u, rtol=1e-6)
    np.testing.assert_allclose(moe.act_fn(g, u, "silu_and_mul_with_clamp"),
                               [0.0, 10 * sig(10.0) * -10, -sig(-1.0) * 2], rtol=1e-6)
    # gelu(0) = 0, gelu(x) -> x for large x, gelu(-1) (tanh form) = -0.15880801
    np.testing.assert_allclose(moe.act_fn(np.array([0.0, 6.0, -1.0], np.float32), np.ones(3, np.float32),
                                          "gelu_tanh"), [0.0, 6.0, -0.15880801], rtol=1e-5, atol=1e-6)


def test_combine_exact_arithmetic():
    """`test_fused_moe_gmm.py:322-384` in spirit: bf16 integer-valued experts,
    inputs and weights 0.125 make every step exact, so the grouped layer must
    equal the per-token loop bit for bit."""
    rng = np.random.default_rng(0)
    T, H, I, E, k = 9, 32, 16, 5, 3
    x = rng.integers(-2, 3, (T, H)).astype(np.float32)
    w13 = rng.integers(-1, 2, (E, 2 * I, H)).astype(np.float32)
    w2 = rng.integers(-1, 2, (E, H, I)).astype(np.float32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[2, 1] = -1
    tw = np.full((T, k), 0.125, np.float32)
    ew = moe.ExpertWeights("bf16", w13, None, w2, None)
    got, _, _ = moe.fused_moe(x, ew, tw, ids, "silu_and_mul_with_clamp")
    want = np.zeros((T, H), np.float32)
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            if e < 0:
                continue
            gu = w13[e] @ x[t]
            a = codecs.bf16_round(moe.act_fn(gu[:I], gu[I:], "silu_and_mul_with_clamp"))
            want[t] += 0.125 * (w2[e] @ a)
    np.testing.assert_allclose(got, codecs.bf16_round(want), rtol=8e-3, atol=1e-6)


def test_grouped_layer_matches_per_token_loop():
    """`_reference_fused_moe`, `test_fused_moe_gmm.py:387-427`: per token and
    slot, skip id < 0, accumulate w * expert(x). Random bf16 data."""
    rng = np.random.default_rng(3)
    T, H, I, E, k = 11, 64, 32, 6, 2
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    w13 = codecs.bf16_round((rng.standard_normal((E, 2 * I, H)) * 0.1).astype(np.float32))
    w2 = codecs.bf16_round((rng.standard_normal((E, H, I)) * 0.1).astype(np.float32))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[0, 0] = -1
    tw = codecs.bf16_round(rng.random((T, k)).astype(np.float32))
    got, _, _ = moe.fused_moe(x, moe.ExpertWeights("bf16", w13, None, w2, None), tw, ids, "silu")
    want = np.zeros((T, H), np.float64)
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            if e >= 0:
                gu = w13[e].astype(np.float64) @ x[t]
                a = codecs.bf16_round(moe.act_fn(gu[:I].astype(np.float32), gu[I:].astype(np.float32), "silu"))
                want[t] += tw[t, j] * (w2[e].astype(np.float64) @ a)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=2e-2 * np.abs(want).max())


def test_fp8_rowquant_expert_linear_is_the_w8a8_recipe():
    """The "fp8_rowquant" expert format's GEMM is the per-channel W8A8 matmul
    of `kernels/quantized_matmul/util.py:80-124` (pinned by its own known
    answers): after the bf16 cast the two agree bit for bit, and a transposed
    scale would not."""
    from oracle import linear, quant

    rng = np.random.default_rng(2)
    E, N, K, R = 3, 48, 64, 5
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    q = [quant.quantize_tensor(w[e], "fp8") for e in range(E)]
    wq, ws = np.stack([a for a, _ in q]), np.stack([b for _, b in q])
    ew = moe.ExpertWeights("fp8_rowquant", wq, ws, wq, ws)
    x = codecs.bf16_round(rng.standard_normal((R, K)).astype(np.float32) * 3)
    for e in range(E):
        ref, _, _ = linear.w8a8_per_channel(x, wq[e], ws[e], "fp8")
        np.testing.assert_array_equal(codecs.bf16_round(ew.linear(13, e, x)), ref)
    assert not np.array_equal(codecs.bf16_round(ew.linear(13, 1, x)),
                              linear.w8a8_per_channel(x, wq[1], ws[0], "fp8")[0])


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_gmm_expert_linear_is_dequantize_then_matmul(fmt):
    """The "fp8" / "int8" expert formats (the grouped matmul's quantized-lhs
    recipe) equal the float64 matmul of the dequantized operands -- the
    activation codes of `quantize_gmm_lhs` (pinned by hand-worked values)
    times their per-(row, 512) scales, the weight codes times their channel
    scales -- to float32 rounding, for each expert."""
    from oracle import quant

    rng = np.random.default_rng(5)
    E, N, K, R = 2, 40, 1536, 4
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    q = [quant.quantize_tensor(w[e], fmt) for e in range(E)]
    wq, ws = np.stack([a for a, _ in q]), np.stack([b for _, b in q])
    ew = moe.ExpertWeights(fmt, wq, ws, wq, ws)
    x = codecs.bf16_round(rng.standard_normal((R, K)).astype(np.float32) * 3)
    x[:, 512:1024] *= 50.0
    xq, xs = quant.quantize_gmm_lhs(x, fmt)
    xd = quant.dequant_codes(xq, fmt).astype(np.float64) * np.repeat(xs, 512, axis=1)
    for e in range(E):
        wd = quant.dequant_codes(wq[e], fmt).astype(np.float64) * ws[e][:, None]
        ref = xd @ wd.T
        np.testing.assert_allclose(ew.linear(13, e, x), ref, rtol=2e-6, atol=2e-6 * np.abs(ref).max())


def test_mx_activation_format_is_two_w4a4_linears():
    """The "mxfp4_mx" expert format on one expert, top 1, routing weight 1:
    the layer is the pinned W4A4 linear of the MX-quantized tokens, the
    activation, a bf16 round, then the W4A4 linear of the MX-quantized
    intermediate (`oracle.linear.w4a4_mxfp4`, `oracle.quant.quantize_mx_fp4`)."""
    from oracle import linear, quant

    rng = np.random.default_rng(4)
    T, H, I = 5, 64, 64
    w13 = rng.integers(0, 256, (1, 2 * I, H // 2), dtype=np.uint8)
    s13 = rng.integers(120, 128, (1, 2 * I, H // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, (1, H, I // 2), dtype=np.uint8)
    s2 = rng.integers(120, 128, (1, H, I // 32), dtype=np.uint8)
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    out, _, _ = moe.fused_moe(x, moe.ExpertWeights("mxfp4_mx", w13, s13, w2, s2), np.ones((T, 1), np.float32),
                              np.zeros((T, 1), np.int32), "swigluoai")
    gu = linear.w4a4_mxfp4(*quant.quantize_mx_fp4(x), w13[0], s13[0])
    a = codecs.bf16_round(moe.act_fn(gu[:, :I], gu[:, I:], "swigluoai"))
    y = linear.w4a4_mxfp4(*quant.quantize_mx_fp4(a), w2[0], s2[0])
    # the layer keeps gate_up in f32 up to the activation; the composition rounds it to bf16 first
    np.testing.assert_allclose(out, y, rtol=2e-2, atol=2e-2 * np.abs(y).max())
    assert not np.array_equal(out, moe.fused_moe(x, moe.ExpertWeights("mxfp4", w13, s13, w2, s2),
                                                 np.ones((T, 1), np.float32), np.zeros((T, 1), np.int32),
                                                 "swigluoai")[0])


def _dense_expert_fixture(i=512, seed=27):
    """The reference's dense-expert fixture (`tests/kernels/experimental/
    test_moe_dense_expert.py:27-37`: m 16, h 512, e 4, randn tokens, integer
    codes in [-8, 8], scales U(0.006, 0.012)) in this package's N-major layout."""
    rng = np.random.default_rng(seed)
    m, h, e = 16, 512, 4
    x = codecs.bf16_round(rng.normal(size=(m, h)).astype(np.float32))
    w13 = codecs.e4m3_encode(rng.integers(-8, 9, size=(e, 2 * i, h)).astype(np.float32))
    w2 = codecs.e4m3_encode(rng.integers(-8, 9, size=(e, h, i)).astype(np.float32))
    s13 = rng.uniform(0.006, 0.012, size=(e, 2 * i)).astype(np.float32)
    s2 = rng.uniform(0.006, 0.012, size=(e, h)).astype(np.float32)
    return x, w13, s13, w2, s2


def dense_expert_case(case):
    """The reference test's routing cases (`test_moe_dense_expert.py:56-70`)
    with its expert-parallel offset 64 removed: ids 64..67 are local experts
    0..3, ids outside them (63, 68, 0..3 before the shift) are -1."""
    ids = np.tile(np.array([[0, 1, -1, -1]], np.int32), (16, 1))
    ids[8:, :2] = [2, 3]
    w = np.tile(np.array([[0.125, 0.25, 0.375, 0.25]], np.float32), (16, 1))
    if case == "single":
        ids[:, :] = [3, -1, -1, -1]
    elif case == "three":
        ids[:, :] = [0, 1, 2, -1]
    elif case == "empty":
        ids[:, :] = -1
    elif case == "zero":
        w[:] = 0
    elif case == "duplicate":
        ids[:, :] = [0, 0, 1, 1]
    return ids, w


@pytest.mark.parametrize("case", ["empty", "zero"])
def test_dense_expert_no_local_work_is_zero(case):
    """Known answer of `test_moe_dense_expert.py:99-101`: no active route
    gives exactly 0."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    ids, w = dense_expert_case(case)
    out = moe.dense_expert_moe(x, w13, s13, w2, s2, w, ids)
    assert np.array_equal(out, np.zeros_like(out))


@pytest.mark.parametrize("i", [512, 640])
@pytest.mark.parametrize("case", ["mixed", "single", "three", "duplicate"])
def test_dense_expert_within_the_reference_bar_of_the_grouped_path(case, i):
    """The reference holds the dense-expert branch to a relative L2 error
    under 0.008 against its grouped path (`test_moe_dense_expert.py:102-104`),
    both with the grouped matmul's bf16 accumulator: here the same bar
    against the grouped oracle with that accumulator (format
    ``fp8_bf16acc``), on the reference's fixture and cases. A dropped
    coefficient, a swapped gate / up half or a transposed weight fails by far.

    Against the f32-accumulated grouped recipe (format ``fp8``, what the
    kernels compute and the north star's fp32-accumulated reference) the gap
    is larger, about 2 % relative L2: the intermediate differs by about 0.5 %
    and its per-(row, 512) e4m3 requantization turns that into fresh rounding
    noise; the north star's cosine bar still holds."""
    x, w13, s13, w2, s2 = _dense_expert_fixture(i)
    ids, w = dense_expert_case(case)
    dense = moe.dense_expert_moe(x, w13, s13, w2, s2, w, ids)
    grouped, _, _ = moe.fused_moe(x, moe.ExpertWeights("fp8_bf16acc", w13, s13, w2, s2), w, ids, "silu")
    rel = np.linalg.norm(dense - grouped) / np.linalg.norm(grouped)
    assert rel < 0.008, rel  # exactly 0 here: the coefficients' products are exact
    f32acc, _, _ = moe.fused_moe(x, moe.ExpertWeights("fp8", w13, s13, w2, s2), w, ids, "silu")
    cos = np.sum(dense * f32acc) / (np.linalg.norm(dense) * np.linalg.norm(f32acc))
    assert cos >= 0.9995 and np.linalg.norm(dense - f32acc) / np.linalg.norm(f32acc) < 0.05


def test_dense_expert_hand_computed_value():
    """One token, one route, every rounding exact: a 448 in the token's block
    gives scale 1 (codes = values); gate code 1 x 16 at scale 1 and up code
    -2 x 14 ... : gate 16, up -28, silu(16) * -28 = -448 in bf16 (sigmoid(16)
    rounds to 1); its block scale is 1 again, the down code 1 at scale 2^-4
    gives -28, times the coefficient 0.5: -14. Gate and up swapped would give
    silu(-28) * 16 ~ 0."""
    h, i, e = 512, 128, 1
    x = np.zeros((1, h), np.float32)
    x[0, 0], x[0, 5] = 448.0, 16.0
    w13 = np.zeros((e, 2 * i, h), np.float32)
    w13[0, 3, 5] = 1.0        # gate channel 3 reads column 5: 16
    w13[0, i + 3, 5] = -1.75  # up channel 3: 16 * -1.75 = -28
    w2 = np.zeros((e, h, i), np.float32)
    w2[0, 7, 3] = 1.0
    s13 = np.ones((e, 2 * i), np.float32)
    s2 = np.full((e, h), 2.0 ** -4, np.float32)
    ids, w = np.array([[0]], np.int32), np.array([[0.5]], np.float32)
    out = moe.dense_expert_moe(x, codecs.e4m3_encode(w13), s13, codecs.e4m3_encode(w2), s2, w, ids)
    expect = np.zeros((1, h), np.float32)
    expect[0, 7] = -14.0
    assert np.array_equal(out, expect)


def test_dense_expert_duplicate_ids_merge_coefficients():
    """Routes of one token to one expert add their coefficients
    (`moe_dense_expert.py:256-262`): ids [0, 0] with weights [a, b] equal
    id 0 with weight a + b when the sum is exact in bf16."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    ids2 = np.tile(np.array([[0, 0]], np.int32), (16, 1))
    w2r = np.tile(np.array([[0.25, 0.5]], np.float32), (16, 1))
    one = moe.dense_expert_moe(x, w13, s13, w2, s2, np.full((16, 1), 0.75, np.float32), ids2[:, :1])
    two = moe.dense_expert_moe(x, w13, s13, w2, s2, w2r, ids2)
    assert np.array_equal(one, two)


def test_dense_expert_nonfinite_expert_stays_with_its_tokens():
    """`test_moe_dense_expert.py:281-304`: with expert 3's gate_up codes NaN,
    tokens routed to expert 0 stay finite, tokens routed to 3 are NaN; a
    zero-coefficient route to expert 3 contributes exactly 0 (the mask)."""
    x, w13, s13, w2, s2 = _dense_expert_fixture()
    w13 = w13.copy()
    w13[3] = 0x7F  # e4m3fn NaN
    ids = np.where(np.arange(16)[:, None] < 8, 0, 3).astype(np.int32)
    with np.errstate(invalid="ignore"):  # the NaN rows' requantization casts NaN
        out = moe.dense_expert_moe(x, w13, s13, w2, s2, np.ones((16, 1), np.float32), ids)
    assert np.isfinite(out[:8]).all() and np.isnan(out[8:]).all()
    ids2 = np.tile(np.array([[0, 3]], np.int32), (16, 1))
    w_zero = np.tile(np.array([[1.0, 0.0]], np.float32), (16, 1))
    masked = moe.dense_expert_moe(x, w13, s13, w2, s2, w_zero, ids2)
    only0 = moe.dense_expert_moe(x, w13, s13, w2, s2, np.ones((16, 1), np.float32), ids2[:, :1])
    assert np.array_equal(masked, only0)
