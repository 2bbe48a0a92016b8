"""GPU parity of the fused decode MoE layer (`qmoe_moe_decode`: shared expert
+ routed experts, `kernels/experimental/fused_moe_decode/
fused_moe_decode_kernel.py:552-740` on one rank) against the CPU oracle
`oracle/decode.py`.

Bars: the north-star row bar against the oracle (the kernel quantizes the
same values the same way; the differences are float32 summation orders,
which can move an intermediate code by one step), and the reference test's
own bar against the decomposed float layer -- max relative row-norm error
below 0.08, with its positive control (dropping one routed expert exceeds
it) -- at the reference test's shapes.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows
from oracle import codecs, decode, quant

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _f8(a, dev):
    return _t(a, dev).view(torch.float8_e4m3fn)


def _q_rows(w):
    s = (np.abs(w).max(axis=-1, keepdims=True) / 448.0).astype(np.float32)
    q = torch.from_numpy(np.ascontiguousarray(w / s)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q, s[..., 0]


def _q_tiles(w):
    """128x128 tiles of [..., N, K] weights (the DeepSeek-V3 checkpoint form)."""
    *lead, n, k = w.shape
    t = w.reshape(*lead, n // 128, 128, k // 128, 128)
    s = (np.abs(t).max(axis=(-3, -1), keepdims=True) / 448.0).astype(np.float32)
    q = torch.from_numpy(np.ascontiguousarray(t / s)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q.reshape(*lead, n, k), s[..., 0, :, 0]


def _layer(seed, E, H, I, Is, T, k, tiles=False, gated=True):
    rng = np.random.default_rng(seed)
    qf = _q_tiles if tiles else _q_rows
    w1q, w1s = qf(rng.standard_normal((E, 2 * I, H), dtype=np.float32) * np.float32(0.02))
    w2q, w2s = qf(rng.standard_normal((E, H, I), dtype=np.float32) * np.float32(0.02))
    sw1q, sw1s = qf(rng.standard_normal((2 * Is, H), dtype=np.float32) * np.float32(0.02))
    sw2q, sw2s = qf(rng.standard_normal((H, Is), dtype=np.float32) * np.float32(0.02))
    gate = codecs.bf16_round((rng.normal(size=H) * 0.02).astype(np.float32)) if gated else None
    x = codecs.bf16_round(rng.normal(size=(T, H)).astype(np.float32))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tw = codecs.bf16_round(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    return dict(hidden=x, w1q=w1q, w1s=w1s, w2q=w2q, w2s=w2s, shared_w1q=sw1q, shared_w1s=sw1s,
                shared_w2q=sw2q, shared_w2s=sw2s, shared_gate=gate, topk_weights=tw, topk_ids=ids,
                weight_blocks=128 if tiles else None)


def _run(L, dev, routed_scale=1.0, tw_dtype=torch.bfloat16):
    from qmoe import ops

    g = L["shared_gate"]
    y = ops.moe_decode(
        _t(L["hidden"], dev, torch.bfloat16), _f8(L["w1q"], dev), _f8(L["w2q"], dev), _t(L["w1s"], dev),
        _t(L["w2s"], dev), _f8(L["shared_w1q"], dev), _t(L["shared_w1s"], dev), _f8(L["shared_w2q"], dev),
        _t(L["shared_w2s"], dev), None if g is None else _t(g, dev, torch.bfloat16),
        _t(L["topk_weights"], dev, tw_dtype), _t(L["topk_ids"], dev), routed_scale=routed_scale,
        weight_blocks=L["weight_blocks"])
    return y.float().cpu().numpy()


def _heaviest(L):
    """Token 0's expert of largest route weight: the positive control drops
    it (the reference test drops ids[0, 0], whose weight may be small)."""
    return int(L["topk_ids"][0, np.argmax(L["topk_weights"][0])])


def _max_rel(a, ref):
    return (np.linalg.norm(a - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)).max()


# (T, E, H, I, Is, k, tiles, gated): T = 1 / 16 / 17 / 64 cross the
# 16-token tile of the down kernel; Is < I; the 128x128-tile variant
CASES = [
    (1, 16, 512, 256, 128, 4, False, True),
    (3, 32, 1024, 512, 256, 6, False, False),
    (8, 64, 1024, 256, 128, 10, False, True),
    (16, 24, 1536, 640, 384, 8, False, True),
    (17, 24, 1024, 384, 384, 4, False, False),
    (40, 64, 512, 256, 256, 8, False, True),
    (64, 16, 1024, 512, 128, 3, False, True),
    (1, 16, 1024, 256, 256, 4, True, False),
    (9, 32, 1024, 512, 256, 6, True, True),
    (33, 16, 512, 256, 128, 4, True, True),
]


@pytest.mark.parametrize("T,E,H,I,Is,k,tiles,gated", CASES)
def test_decode_matches_oracle(dev, T, E, H, I, Is, k, tiles, gated):
    print(f"moe_decode T={T} E={E} H={H} I={I} Is={Is} k={k} tiles={tiles} gated={gated}", flush=True)
    L = _layer(T * 7 + E, E, H, I, Is, T, k, tiles, gated)
    got = _run(L, dev)
    ref = decode.fused_moe_decode(**L)
    assert_close_rows(got, ref, "moe_decode vs oracle", rel=1e-2)
    assert _max_rel(got, decode.decomposed_layer_f32(**L)) < 0.08


@pytest.mark.parametrize("m,padded", [(8, False), (8, True), (32, False)])
def test_reference_decomposed_layer_bar(dev, m, padded):
    """`test_fused_moe_decode_kernel.py:280-296` at its shapes (H 1024, I
    256, I_s 128, E 64, top-10, gated shared expert)."""
    print(f"moe_decode reference bar m={m} padded={padded}", flush=True)
    L = _layer(m, 64, 1024, 256, 128, m, 10)
    if padded:
        L["topk_weights"][m - 3:] = 0.0
    got = _run(L, dev)
    ref = decode.decomposed_layer_f32(**L)
    assert np.isfinite(got).all()
    assert _max_rel(got, ref) < 0.08
    broken = decode.decomposed_layer_f32(**L, skip_expert=_heaviest(L))
    assert _max_rel(got, broken) > 0.08
    assert_close_rows(got, decode.fused_moe_decode(**L), "vs oracle", rel=1e-2)


def test_ungated_routed_scale_and_f32_weights(dev):
    """GLM convention (ungated shared expert, routed_scale 2.5 on the routed
    sum only), route weights handed over as float32 (rounded to bf16 first,
    as the reference casts them to the activation dtype)."""
    print("moe_decode ungated routed_scale 2.5", flush=True)
    L = _layer(5, 64, 1024, 256, 128, 8, 10, gated=False)
    L["topk_weights"] = np.random.default_rng(1).dirichlet(np.ones(10), size=8).astype(np.float32)
    got = _run(L, dev, routed_scale=2.5, tw_dtype=torch.float32)
    assert_close_rows(got, decode.fused_moe_decode(**L, routed_scale=2.5), "routed_scale", rel=1e-2)
    ref = decode.decomposed_layer_f32(**L, routed_scale=2.5)
    assert _max_rel(got, ref) < 0.08
    shared_only = decode.decomposed_layer_f32(**{**L, "topk_weights": np.zeros_like(L["topk_weights"])})
    assert _max_rel(got, ref + 1.5 * shared_only) > 0.08


def test_duplicate_invalid_and_zero_routes(dev):
    """Ids outside [0, E) select nothing, a token naming an expert twice
    sums the two weights into one row, zero-weight routes add nothing, and
    a token with no valid route gets the shared expert alone."""
    print("moe_decode edge routes", flush=True)
    L = _layer(21, 12, 512, 256, 256, 6, 4)
    ids = L["topk_ids"]
    ids[0, 1] = ids[0, 0]   # duplicate
    ids[1, 2] = -1          # invalid
    ids[2, 3] = 12          # invalid (== E)
    L["topk_weights"][3, 1] = 0.0
    ids[4, :] = -1          # no routed expert
    L["topk_weights"][5, :] = 0.0
    got = _run(L, dev)
    ref = decode.fused_moe_decode(**L)
    assert_close_rows(got, ref, "edge routes", rel=1e-2)
    shared_only = decode.fused_moe_decode(**{**L, "topk_weights": np.zeros_like(L["topk_weights"])})
    np.testing.assert_array_equal(got[4], _run({**L, "topk_weights": np.zeros_like(L["topk_weights"])}, dev)[4])
    assert_close_rows(got[4:6], shared_only[4:6], "shared only", rel=1e-2)


def test_repeat_calls_are_deterministic(dev):
    """Row positions inside a group vary between calls (LDS atomics); each
    row is computed on its own and the per-token sum runs in slot order, so
    repeated calls agree bit for bit."""
    L = _layer(3, 32, 1024, 512, 256, 12, 8)
    a = _run(L, dev)
    for _ in range(3):
        np.testing.assert_array_equal(_run(L, dev), a)


@pytest.mark.parametrize("T,tiles", [(40, False), (64, True)])
def test_split_down_ranges(dev, T, tiles):
    """Above 16 tokens the down kernel cuts the active list into ranges
    whose partial sums a last launch adds in range order: repeated calls
    agree bit for bit, tokens with no valid route (and a step whose routes
    are all invalid: one active slot, the shared expert) get the shared
    expert alone, and the result meets the oracle bar."""
    print(f"moe_decode split down T={T} tiles={tiles}", flush=True)
    L = _layer(T + 5, 48, 1024, 256, 128, T, 6, tiles=tiles)
    L["topk_ids"][3, :] = -1
    L["topk_ids"][T - 1, :] = 48
    a = _run(L, dev)
    for _ in range(2):
        np.testing.assert_array_equal(_run(L, dev), a)
    assert_close_rows(a, decode.fused_moe_decode(**L), f"split down T={T}", rel=1e-2)
    # shared expert alone (I_s = 128): a row of small values, where one
    # intermediate code on the other side of a rounding boundary is a few
    # bf16 ulps -- the north-star row bar
    none = {**L, "topk_ids": np.full_like(L["topk_ids"], -1)}
    assert_close_rows(_run(none, dev), decode.fused_moe_decode(**none), "no routed expert")


# (T, E, k, scoring, groups, bias, tiles): T <= 8 routes inside the prep
# launch (1, 2, 4 and 8 slots per row, group sizes 32, 16, 64 and 20), T > 8
# through the router's own launch first
ROUTED_CASES = [
    (1, 256, 8, "sigmoid", (8, 4), True, True),
    (3, 128, 4, "softmax", None, False, False),
    (8, 64, 6, "sqrtsoftplus", None, True, True),
    (5, 320, 6, "sigmoid", (5, 2), True, False),
    (2, 160, 6, "softmax", (8, 3), False, True),
    (6, 96, 4, "sigmoid", (6, 3), True, False),
    (12, 96, 4, "softmax", (6, 3), False, True),
]


@pytest.mark.parametrize("T,E,k,scoring,groups,use_bias,tiles", ROUTED_CASES)
def test_decode_routed_matches_route_then_decode(dev, T, E, k, scoring, groups, use_bias, tiles):
    """`moe_decode_routed` (the op routes the tokens itself) gives bit for
    bit the routes of `moe_route` and the output of `moe_decode` on them."""
    from qmoe import ops

    print(f"moe_decode_routed T={T} E={E} k={k} {scoring} groups={groups} bias={use_bias} tiles={tiles}",
          flush=True)
    H, I, Is = 1024, 256, 128
    L = _layer(T * 13 + E, E, H, I, Is, T, k, tiles=tiles, gated=True)
    rng = np.random.default_rng(E + T)
    logits = _t(codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32)), dev, torch.bfloat16)
    bias = _t((rng.standard_normal(E) * 0.1).astype(np.float32), dev) if use_bias else None
    ng, tg = groups if groups else (1, 1)
    rkw = dict(bias=bias, routed_scaling_factor=1.5 if use_bias else 1.0, num_expert_group=ng, topk_group=tg)
    g = _t(L["shared_gate"], dev, torch.bfloat16)
    wts = (_f8(L["w1q"], dev), _f8(L["w2q"], dev), _t(L["w1s"], dev), _t(L["w2s"], dev),
           _f8(L["shared_w1q"], dev), _t(L["shared_w1s"], dev), _f8(L["shared_w2q"], dev),
           _t(L["shared_w2s"], dev), g)
    x = _t(L["hidden"], dev, torch.bfloat16)
    wr, ir = ops.moe_route(logits, k, scoring, True, **rkw)
    yr = ops.moe_decode(x, *wts, wr, ir, routed_scale=2.5, weight_blocks=L["weight_blocks"])
    y, w, ids = ops.moe_decode_routed(x, logits, k, *wts, scoring_func=scoring, renormalize=True, **rkw,
                                      routed_scale=2.5, weight_blocks=L["weight_blocks"])
    np.testing.assert_array_equal(ids.cpu().numpy(), ir.cpu().numpy())
    np.testing.assert_array_equal(w.view(torch.int16).cpu().numpy(), wr.view(torch.int16).cpu().numpy())
    np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy(), yr.view(torch.int16).cpu().numpy())


@pytest.mark.parametrize("T,tiles", [(1, True), (1, False), (8, True), (16, False)])
def test_decode_deepseek_v3_shapes(dev, T, tiles):
    """BASELINE config 4's layer (E 256, H 7168, I 2048, top-8, one shared
    expert of the same size), weights generated on the device; only the
    experts the tokens touch are copied to the host for the oracle."""
    from qmoe import ops

    print(f"moe_decode dsv3 T={T} tiles={tiles}", flush=True)
    E, H, I, k = 256, 7168, 2048, 8
    gen = torch.Generator(device=dev).manual_seed(T + 2 * tiles)

    def qdev(shape):
        w = torch.randn(shape, device=dev, generator=gen) * 0.02
        if tiles:
            *lead, n, kk = shape
            t = w.reshape(*lead, n // 128, 128, kk // 128, 128)
            s = t.abs().amax(dim=(-3, -1), keepdim=True) / 448.0
            return (t / s).to(torch.float8_e4m3fn).reshape(shape), s[..., 0, :, 0].contiguous()
        s = w.abs().amax(dim=-1, keepdim=True) / 448.0
        return (w / s).to(torch.float8_e4m3fn), s[..., 0].contiguous()

    w1, s1 = zip(*[qdev((2 * I, H)) for _ in range(E)])
    w1, s1 = torch.stack(w1), torch.stack(s1)
    w2, s2 = zip(*[qdev((H, I)) for _ in range(E)])
    w2, s2 = torch.stack(w2), torch.stack(s2)
    sw1, ss1 = qdev((2 * I, H))
    sw2, ss2 = qdev((H, I))
    rng = np.random.default_rng(T)
    x = codecs.bf16_round(rng.normal(size=(T, H)).astype(np.float32))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tw = codecs.bf16_round(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    got = ops.moe_decode(_t(x, dev, torch.bfloat16), w1, w2, s1, s2, sw1, ss1, sw2, ss2, None,
                         _t(tw, dev, torch.bfloat16), _t(ids, dev), routed_scale=2.5,
                         weight_blocks=128 if tiles else None).float().cpu().numpy()
    touched = np.unique(ids)
    remap = {int(e): i for i, e in enumerate(touched)}
    u8 = lambda t: t.view(torch.uint8).cpu().numpy()  # noqa: E731
    sel = torch.from_numpy(touched).to(dev)
    L = dict(hidden=x, w1q=u8(w1[sel]), w1s=s1[sel].cpu().numpy(), w2q=u8(w2[sel]), w2s=s2[sel].cpu().numpy(),
             shared_w1q=u8(sw1), shared_w1s=ss1.cpu().numpy(), shared_w2q=u8(sw2), shared_w2s=ss2.cpu().numpy(),
             shared_gate=None, topk_weights=tw, topk_ids=np.vectorize(remap.get)(ids).astype(np.int32),
             weight_blocks=128 if tiles else None)
    ref = decode.fused_moe_decode(**L, routed_scale=2.5)
    assert_close_rows(got, ref, f"dsv3 T={T}", rel=1e-2)


def _armed_runner(dev, monkeypatch, E, H, I, Is, k, gated, rsf, seed):
    """A MoE runner as vLLM builds it (routed layer + shared MLP), loaded
    from a per-channel FP8 checkpoint through the quant methods."""
    import types

    from qmoe.layers import quantization as q

    for v in ("MOE_REQUANTIZE_WEIGHT_DTYPE", "MOE_REQUANTIZE_BLOCK_SIZE", "QMOE_FP8_NATIVE_BLOCKS",
              "REQUANTIZE_BLOCK_SIZE", "ENABLE_QUANTIZED_MATMUL_KERNEL"):
        monkeypatch.delenv(v, raising=False)
    rng = np.random.default_rng(seed)
    cfg = q.Fp8Config(is_checkpoint_fp8_serialized=False)  # bf16 weights, quantized at load
    layer = torch.nn.Module()
    layer.moe_config = types.SimpleNamespace(experts_per_token=k, has_bias=False)
    layer.renormalize, layer.scoring_func = True, "softmax"
    layer.e_score_correction_bias, layer.use_grouped_topk = None, False
    layer.routed_scaling_factor, layer.custom_routing_function = 1.0, None
    layer.activation = "silu"
    method = q.Fp8MoEMethod(cfg, layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    layer.w13_weight.data = _t(rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.02, dev, torch.bfloat16)
    layer.w2_weight.data = _t(rng.standard_normal((E, H, I)).astype(np.float32) * 0.02, dev, torch.bfloat16)
    method.process_weights_after_loading(layer)

    def linear(n, kk):
        lm = q.Fp8LinearMethod(cfg)
        lin = torch.nn.Module()
        lm.create_weights(lin, kk, [n], kk, n, torch.bfloat16)
        lin.weight.data = _t(rng.standard_normal((n, kk)).astype(np.float32) * 0.02, dev, torch.bfloat16)
        lm.process_weights_after_loading(lin)
        return lin

    mlp = torch.nn.Module()
    mlp.gate_up_proj, mlp.down_proj = linear(2 * Is, H), linear(H, Is)
    mlp.expert_gate = None
    if gated:
        g = torch.nn.Module()
        g.weight = torch.nn.Parameter(_t(rng.standard_normal((1, H)).astype(np.float32) * 0.02, dev,
                                         torch.bfloat16), requires_grad=False)
        g.bias = None
        mlp.expert_gate = g
    runner = torch.nn.Module()
    runner.routed_experts = layer
    runner._quant_method = method
    runner._shared_experts = types.SimpleNamespace(_layer=mlp)
    runner.routed_scaling_factor = rsf
    runner.moe_config = layer.moe_config
    model = torch.nn.Module()
    model.runner = runner
    return model, runner, layer, method, mlp


def _layer_oracle(layer, mlp, x, logits, k, rsf, gated):
    """The decode recipe on the processed weights, routed by the oracle."""
    from oracle import routing

    u8 = lambda t: t.view(torch.uint8).cpu().numpy()  # noqa: E731
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    gate = None if not gated else f(mlp.expert_gate.weight).reshape(-1)
    L = dict(hidden=x, w1q=u8(layer.w13_weight), w1s=f(layer.w13_weight_scale), w2q=u8(layer.w2_weight),
             w2s=f(layer.w2_weight_scale), shared_w1q=u8(mlp.gate_up_proj.weight),
             shared_w1s=f(mlp.gate_up_proj.weight_scale).reshape(-1), shared_w2q=u8(mlp.down_proj.weight),
             shared_w2s=f(mlp.down_proj.weight_scale).reshape(-1), shared_gate=gate, topk_weights=tw,
             topk_ids=ids)
    return decode.fused_moe_decode(**L, routed_scale=rsf), L


@pytest.mark.parametrize("gated,rsf", [(True, 1.0), (False, 2.5)])
def test_armed_layer_serves_shared_plus_routed(dev, monkeypatch, gated, rsf):
    """`arm_fused_moe_decode` on a runner (Fp8 MoE method, per-channel
    experts, FP8 shared MLP): the runner loses its shared expert and its
    routed_scaling_factor (now the op's), and `apply_monolithic` returns
    shared + routed from the fused decode op (`fused_moe_decode.py:513-649`).
    Above FUSED_MOE_DECODE_KERNEL_MAX_TOKENS the same call runs the GMM MoE
    plus the shared linears."""
    from qmoe.layers import fused_moe_decode as fmd

    print(f"armed layer gated={gated} rsf={rsf}", flush=True)
    monkeypatch.setenv("FUSED_MOE_DECODE_KERNEL", "1")
    monkeypatch.setenv("FUSED_MOE_DECODE_KERNEL_MAX_TOKENS", "8")
    E, H, I, Is, k = 16, 512, 256, 128, 4
    model, runner, layer, method, mlp = _armed_runner(dev, monkeypatch, E, H, I, Is, k, gated, rsf, seed=4)
    assert fmd.arm_fused_moe_decode(model) == 1
    assert runner._shared_experts is None and runner.routed_scaling_factor == 1.0
    assert fmd.fused_moe_decode_supported(method)
    rng = np.random.default_rng(9)
    for T in (5, 11):  # 11 > the cap of 8: the GMM path
        x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
        logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
        got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
        ref, L = _layer_oracle(layer, mlp, x, logits, k, rsf, gated)
        if T <= 8:
            # the op routed the tokens itself: bit-equal to routing first
            from qmoe.layers import moe_routing

            xt, lt = _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16)
            tw, ti = moe_routing.route(layer, xt, lt)
            two = fmd.fused_moe_decode(method, layer, xt, tw, ti)
            np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(), two.view(torch.int16).cpu().numpy())
        got = got.float().cpu().numpy()
        if T <= 8:
            assert_close_rows(got, ref, f"armed T={T}", rel=1e-2)
        else:
            # a different recipe (the GMM MoE's and the dense linears'):
            # the reference test's bar against the decomposed layer
            assert _max_rel(got, decode.decomposed_layer_f32(**L, routed_scale=rsf)) < 0.08


def test_arming_caps_the_op_at_the_measured_crossover(dev, monkeypatch):
    """Above QMOE_DECODE_OP_MAX_TOKENS (16: the fused op's measured
    crossover with the GMM path) an armed layer's steps take the GMM path
    even under a larger FUSED_MOE_DECODE_KERNEL_MAX_TOKENS; 0 leaves the
    reference's cap alone."""
    from qmoe.layers import fused_moe_decode as fmd

    print("decode op crossover cap", flush=True)
    monkeypatch.setenv("FUSED_MOE_DECODE_KERNEL", "1")
    monkeypatch.setenv("FUSED_MOE_DECODE_KERNEL_MAX_TOKENS", "64")
    for env, cap in ((None, 16), ("0", 64), ("4", 4)):
        if env is None:
            monkeypatch.delenv("QMOE_DECODE_OP_MAX_TOKENS", raising=False)
        else:
            monkeypatch.setenv("QMOE_DECODE_OP_MAX_TOKENS", env)
        model, _, _, method, _ = _armed_runner(dev, monkeypatch, 8, 512, 128, 128, 2, False, 1.0, seed=5)
        assert fmd.arm_fused_moe_decode(model) == 1
        assert getattr(method, fmd.FUSED_MOE_DECODE_OP_ATTR)["max_tokens"] == cap
