"""GPU parity at the BASELINE configs' own shapes.

Every config point that bench.py times runs here through the same entry
points (the reference's op functions `quantized_matmul`, `quantized_matmul_fp4`
and the MoE layer), on full-size seeded inputs; a strided sample of output
rows (tokens) is checked against the oracle:

* integer work bit-exactly: activation codes and scales of the sampled rows,
  routing ids of every token, INT8 GEMM outputs;
* same-code FP8 / e2m1 GEMMs within one bf16 ulp (the operands are exact in
  f32, only the summation order differs);
* MoE layers (which re-quantize the bf16 intermediate, so codes can differ at
  rounding boundaries) within the north-star bar, max |err| <= 2e-2 * row max
  and cosine >= 0.9995.

Weights are generated on the device (seeded) and only what the oracle needs
(the weight set of a linear, the experts that the sampled tokens route to)
is copied to the host. The module records the kernel plan (path, token tile,
K split) of every GEMM it runs; its last test asserts that each plan the
benchmark's config points use is among them.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows, assert_close_same_codes
from oracle import codecs, linear, quant, routing
from oracle import moe as omoe

pytestmark = pytest.mark.gpu

_PLANS = set()  # kernel plans exercised by this module's tests


def _rows_sample(M, n=40):
    """Strided row sample: n rows spread over [0, M) at varying offsets
    inside each stride (so every token tile and positions inside tiles are
    hit), plus the first and last row."""
    if M <= n:
        return np.arange(M)
    stride = M // n
    r = [i * stride + (i * 37) % stride for i in range(n)] + [0, M - 1]
    return np.unique(np.asarray(r))


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _np(t):
    return t.cpu().numpy()


def _run(fn):
    from qmoe import ops

    with ops.record_plans() as plans:
        out = fn()
    _PLANS.update(plans)
    return out


# ------------------------------------------------------------------ config 1

_W1 = {}


def _cfg1_weights(qd, K, N):
    """randn * 0.02 weights quantized per channel at load time (the device
    quantizer, bit-exact with the oracle's `quantize_tensor`, which is checked
    on a sample of weight rows here)."""
    from qmoe import ops

    key = (qd, K, N)
    if key not in _W1:
        _W1.clear()
        g = _gen(100 + K)
        w = torch.randn((N, K), device="cuda", generator=g) * 0.02
        q, s = ops.row_quant(w, qd, mode="load")
        rows = _rows_sample(N, 8)
        q_ref, s_ref = quant.quantize_tensor(_np(w[rows]), qd)
        np.testing.assert_array_equal(_np(q[rows].view(torch.uint8)), q_ref.view(np.uint8))
        np.testing.assert_array_equal(_np(s[rows]), s_ref)
        del w
        _W1[key] = (q, s, _np(q.view(torch.uint8)), _np(s))
    return _W1[key]


@pytest.mark.parametrize("M", [1, 8, 64, 512, 4096])
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("qd", ["fp8", "int8"])
def test_cfg1_w8a8_per_channel(dev, qd, K, N, M):
    """Config 1: per-token dynamic quant + per-channel W8A8 at the Llama-3-8B
    MLP shapes, through `quantized_matmul` (the 256-token tiles at M = 4096
    and the 128-token tiles at M = 512 included)."""
    from qmoe import ops
    from qmoe.layers.linear_common import quantized_matmul

    print(f"cfg1 {qd} M={M} K={K} N={N}", flush=True)
    q, s, wq, ws = _cfg1_weights(qd, K, N)
    x = torch.randn((M, K), device="cuda", generator=_gen(M + K)).to(torch.bfloat16)
    y = _run(lambda: quantized_matmul(x, q.t(), s))
    rows = _rows_sample(M)
    xr = _np(x[rows].float())
    xq, xs = ops.row_quant(x, qd)
    ref, xq_ref, xs_ref = linear.w8a8_per_channel(xr, wq.view(np.int8) if qd == "int8" else wq, ws, qd)
    np.testing.assert_array_equal(_np(xq[rows].view(torch.uint8)), xq_ref.view(np.uint8))
    np.testing.assert_array_equal(_np(xs[rows]), xs_ref)
    got = _np(y[rows].float())
    if qd == "int8":
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_same_codes(got, ref, f"cfg1 fp8 {M}x{K}x{N}")


# ------------------------------------------------------------------ config 2

_W2 = {}


def _tile_weights(N, K, g):
    """randn * 0.02 weights in the DeepSeek-V3 checkpoint form: e4m3 codes
    and one f32 scale_inv per 128 x 128 tile (device torch ops)."""
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    t = w.view(N // 128, 128, K // 128, 128)
    s = t.abs().amax(dim=(1, 3)) / 448.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    q = (t / s[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(N, K)
    return q, s.float().contiguous()


@pytest.mark.parametrize("M", [1, 32, 256, 2048, 8192])
@pytest.mark.parametrize("N", [18432, 24576])
def test_cfg2_fp8_block128(dev, N, M):
    """Config 2: 128 x 128 block-scaled FP8 weights, activations quantized per
    (token, 128 columns), K = 7168, through `quantized_matmul` with the
    compact tile scales."""
    from qmoe import ops
    from qmoe.layers.linear_common import quantized_matmul

    K = 7168
    print(f"cfg2 M={M} K={K} N={N}", flush=True)
    if N not in _W2:
        _W2.clear()
        q, s = _tile_weights(N, K, _gen(200 + N))
        _W2[N] = (q, s, _np(q.view(torch.uint8)), _np(s))
    q, s, wq, st = _W2[N]
    x = torch.randn((M, K), device="cuda", generator=_gen(M + N)).to(torch.bfloat16)
    y = _run(lambda: quantized_matmul(x, q.t(), s))
    rows = _rows_sample(M, 24)
    xr = _np(x[rows].float())
    xq, xs = ops.row_quant(x, "fp8", block=128)
    ref, xq_ref, xs_ref = linear.w8a8_blockwise(xr, wq, linear.tile_scales_to_blocks(st, N))
    np.testing.assert_array_equal(_np(xq[rows].view(torch.uint8)), xq_ref)
    np.testing.assert_array_equal(_np(xs[rows]), xs_ref)
    assert_close_same_codes(_np(y[rows].float()), ref, f"cfg2 {M}x{K}x{N}")


# ------------------------------------------------------------------ config 0


@pytest.mark.parametrize("M", [1, 16, 128, 2048, 8192])
def test_cfg0_mxfp4(dev, M):
    """Config 0: MXFP4 weights (uniform e2m1 codes, e8m0 exponents in
    [-8, 0]) x bf16 activations, K = 2880, N = 5760, through
    `quantized_matmul_fp4` (M 2048 / 8192: the large-M tiles)."""
    from qmoe.layers.linear_common import quantized_matmul_fp4

    K, N = 2880, 5760
    print(f"cfg0 M={M}", flush=True)
    g = _gen(300)
    codes = torch.randint(0, 256, (N, K // 2), device="cuda", dtype=torch.uint8, generator=g)
    sc = (127 + torch.randint(-8, 1, (N, K // 32), device="cuda", generator=g)).to(torch.uint8)
    x = torch.randn((M, K), device="cuda", generator=_gen(M)).to(torch.bfloat16)
    y = _run(lambda: quantized_matmul_fp4(x, codes, sc))
    rows = _rows_sample(M)
    ref = linear.w4a16_mxfp4(_np(x[rows].float()), _np(codes), _np(sc))
    assert_close_same_codes(_np(y[rows].float()), ref, f"cfg0 M={M}")


# ------------------------------------------------------------------ MoE


class _DeviceExperts:
    """[E, ...] device tensor read one expert at a time (the oracle's
    `ExpertWeights` indexes w[e])."""

    def __init__(self, t):
        self.t = t
        self.shape = tuple(t.shape)

    def __getitem__(self, e):
        return _np(self.t[int(e)])


def _layer_cfg(topk, scoring, activation, bias=None, rsf=1.0, groups=None):
    from types import SimpleNamespace

    return SimpleNamespace(moe_config=SimpleNamespace(experts_per_token=topk), scoring_func=scoring,
                           renormalize=True, e_score_correction_bias=bias, routed_scaling_factor=rsf,
                           use_grouped_topk=groups is not None, num_expert_group=groups[0] if groups else 1,
                           topk_group=groups[1] if groups else 1, custom_routing_function=None,
                           _qmoe_activation=activation)


_E3 = {}


def _cfg3_experts(bias):
    if "w" not in _E3:
        E, H, I = 128, 2880, 2880
        g = _gen(400)
        w13 = torch.randint(0, 256, (E, 2 * I, H // 2), device="cuda", dtype=torch.uint8, generator=g)
        s13 = (127 + torch.randint(-8, 1, (E, 2 * I, H // 32), device="cuda", generator=g)).to(torch.uint8)
        w2 = torch.randint(0, 256, (E, H, I // 2), device="cuda", dtype=torch.uint8, generator=g)
        s2 = (127 + torch.randint(-8, 1, (E, H, I // 32), device="cuda", generator=g)).to(torch.uint8)
        b13 = torch.randn((E, 2 * I), device="cuda", generator=g) * 0.1
        b2 = torch.randn((E, H), device="cuda", generator=g) * 0.1
        _E3["w"] = (w13, s13, w2, s2, b13, b2)
    w13, s13, w2, s2, b13, b2 = _E3["w"]
    return (w13, s13, w2, s2) + ((b13, b2) if bias else (None, None))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("T", [1, 16, 128, 1024, 8192])
def test_cfg3_gptoss_moe(dev, T, bias):
    """Config 3: GPT-OSS-120B-shaped MXFP4 MoE (E 128, top 4, H = I = 2880,
    softmax over the top 4, swigluoai), the layer as a MoE method runs it
    (`moe_forward`: fused route + dispatch up to 16 tokens), with and without
    the checkpoint's expert biases. Routing ids of every token are checked
    bit-exactly; the layer output on a token sample."""
    from qmoe import ops
    from qmoe.layers.fused_moe import moe_forward

    E, k, H = 128, 4, 2880
    print(f"cfg3 T={T} bias={bias}", flush=True)
    w13, s13, w2, s2, b13, b2 = _cfg3_experts(bias)
    g = _gen(410 + T)
    x = torch.randn((T, H), device="cuda", generator=g).to(torch.bfloat16)
    logits = torch.randn((T, E), device="cuda", generator=g).to(torch.bfloat16)
    lc = _layer_cfg(k, "softmax", "swigluoai")
    y = _run(lambda: moe_forward(lc, x, logits, w13, w2, s13, s2, b13, b2, "mxfp4"))
    tw, ids = ops.moe_route(logits, k, "softmax", True)
    w_ref, ids_ref = routing.select_experts(_np(logits.float()), k, True, "softmax")
    np.testing.assert_array_equal(_np(ids), ids_ref)
    toks = _rows_sample(T, 4)
    ew = omoe.ExpertWeights("mxfp4", _DeviceExperts(w13), _DeviceExperts(s13), _DeviceExperts(w2),
                            _DeviceExperts(s2), _DeviceExperts(b13) if bias else None,
                            _DeviceExperts(b2) if bias else None, keep=False)
    ref = omoe.fused_moe_tokens(_np(x[toks].float()), ew, _np(tw[toks].float()), ids_ref[toks], "swigluoai", E)
    assert_close_rows(_np(y[toks].float()), ref, f"cfg3 T={T}")


_E4 = {}


def _cfg4_experts():
    """256 routed experts + 1 shared in the 128 x 128 FP8 checkpoint form
    (11.3 GB), generated on the device once per module."""
    if "w" not in _E4:
        E, H, I = 256, 7168, 2048
        g = _gen(500)
        w13 = torch.empty((E, 2 * I, H), device="cuda", dtype=torch.float8_e4m3fn)
        s13 = torch.empty((E, 2 * I // 128, H // 128), device="cuda", dtype=torch.float32)
        w2 = torch.empty((E, H, I), device="cuda", dtype=torch.float8_e4m3fn)
        s2 = torch.empty((E, H // 128, I // 128), device="cuda", dtype=torch.float32)
        for e in range(E):
            w13[e], s13[e] = _tile_weights(2 * I, H, g)
            w2[e], s2[e] = _tile_weights(H, I, g)
        sh13, ss13 = _tile_weights(2 * I, H, g)
        sh2, ss2 = _tile_weights(H, I, g)
        bias = torch.randn(E, device="cuda", generator=g) * 0.1
        _E4["w"] = (w13, s13, w2, s2, sh13, ss13, sh2, ss2, bias)
    return _E4["w"]


def _cfg4_logits(T, skew, g):
    E = 256
    logits = torch.randn((T, E), device="cuda", generator=g)
    if skew:
        # 30% of tokens: +8 on 8 hot experts, 2 per group in groups 0-3
        hot = torch.tensor([0, 1, 32, 33, 64, 65, 96, 97], device="cuda")
        sel = torch.rand(T, device="cuda", generator=g) < 0.3
        if T == 1:
            sel[0] = True
        logits[sel.nonzero()[:, 0][:, None], hot[None, :]] += 8.0
    return logits.to(torch.bfloat16)


@pytest.mark.parametrize("skew", [False, True])
@pytest.mark.parametrize("T", [1, 8, 64, 512, 4096])
def test_cfg4_deepseek_moe(dev, T, skew):
    """Config 4: DeepSeek-V3-shaped routed experts (E 256, top 8 of 4 of 8
    groups, sigmoid scores with a correction bias, routed_scaling_factor 2.5,
    silu), 128 x 128 block-scaled FP8 with per-(token, 128) activation quant,
    through `moe_forward`; the skewed variant sends 30% of tokens to 8 hot
    experts. Ids of every token bit-exact; layer output on a token sample."""
    from qmoe import ops
    from qmoe.layers.fused_moe import moe_forward

    E, k, H = 256, 8, 7168
    print(f"cfg4 T={T} skew={skew}", flush=True)
    w13, s13, w2, s2, _, _, _, _, bias = _cfg4_experts()
    g = _gen(510 + T + skew)
    x = torch.randn((T, H), device="cuda", generator=g).to(torch.bfloat16)
    logits = _cfg4_logits(T, skew, g)
    lc = _layer_cfg(k, "sigmoid", "silu", bias=bias, rsf=2.5, groups=(8, 4))
    y = _run(lambda: moe_forward(lc, x, logits, w13, w2, s13, s2, None, None, "fp8_block"))
    tw, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5,
                            num_expert_group=8, topk_group=4)
    _, ids_ref = routing.grouped_topk(_np(logits.float()), k, True, 8, 4, "sigmoid", _np(bias), 2.5)
    np.testing.assert_array_equal(_np(ids), ids_ref)
    if skew and T >= 64:
        # the load imbalance is there: the 8 hot experts take at least 3x
        # their uniform share of the routes (the correction bias keeps the
        # boosted tokens from landing on exactly the hot set every time)
        cnt = np.bincount(ids_ref.reshape(-1), minlength=E)
        hot = cnt[[0, 1, 32, 33, 64, 65, 96, 97]].sum()
        assert hot >= 3 * T * k * 8 / E, (hot, T)
    toks = _rows_sample(T, 3)
    ew = omoe.ExpertWeights("fp8_block", _DeviceExperts(w13.view(torch.uint8)), _DeviceExperts(s13),
                            _DeviceExperts(w2.view(torch.uint8)), _DeviceExperts(s2), keep=False)
    ref = omoe.fused_moe_tokens(_np(x[toks].float()), ew, _np(tw[toks].float()), ids_ref[toks], "silu", E)
    assert_close_rows(_np(y[toks].float()), ref, f"cfg4 T={T} skew={skew}")


@pytest.mark.parametrize("T", [1, 8, 64, 512, 4096])
def test_cfg4_shared_expert(dev, T):
    """Config 4's shared expert: the block-scaled gate_up GEMM with the silu
    fused (N = 2 x 2048, K = 7168), the intermediate re-quantized per (token,
    128), and the down GEMM (N = 7168, K = 2048)."""
    from qmoe import _capi, ops

    I, H = 2048, 7168
    print(f"cfg4 shared T={T}", flush=True)
    _, _, _, _, sh13, ss13, sh2, ss2, _ = _cfg4_experts()
    x = torch.randn((T, H), device="cuda", generator=_gen(520 + T)).to(torch.bfloat16)

    def shared():
        xq, xs = ops.row_quant(x, "fp8", block=128)
        a = ops.gemm(_capi.W8A8_BLK, xq.view(torch.uint8), sh13.view(torch.uint8), a_scale=xs, w_scale=ss13,
                     ws_bn=128, activation="silu")
        aq, as_ = ops.row_quant(a, "fp8", block=128)
        return a, ops.gemm(_capi.W8A8_BLK, aq.view(torch.uint8), sh2.view(torch.uint8), a_scale=as_,
                           w_scale=ss2, ws_bn=128)

    a, y = _run(shared)
    toks = _rows_sample(T, 16)
    w13n, s13n = _np(sh13.view(torch.uint8)), _np(ss13)
    gu, _, _ = linear.w8a8_blockwise(_np(x[toks].float()), w13n, linear.tile_scales_to_blocks(s13n, 2 * I),
                                     round_out=False)
    a_ref = codecs.bf16_round(omoe.act_fn(gu[:, :I], gu[:, I:], "silu"))
    assert_close_rows(_np(a[toks].float()), a_ref, f"cfg4 shared gate_up T={T}")
    # the down projection of the device's own intermediate: same codes
    ref, _, _ = linear.w8a8_blockwise(_np(a[toks].float()), _np(sh2.view(torch.uint8)),
                                      linear.tile_scales_to_blocks(_np(ss2), H))
    assert_close_same_codes(_np(y[toks].float()), ref, f"cfg4 shared down T={T}")


_E4D = {}


def _cfg4_default_layer(qd):
    """Config 4's checkpoint through the FP8 MoE method's default load path
    (`fp8.py:486-617`: 128 x 128 tiles dequantized in float32 on the
    device, requantized per output channel to e4m3, or to int8 with
    MOE_REQUANTIZE_WEIGHT_DTYPE=int8); one processed layer kept at a time."""
    import types

    from qmoe.layers import quantization as q

    if _E4D.get("qd") != qd:
        _E4D.clear()
        import os

        w13, s13, w2, s2, _, _, _, _, bias = _cfg4_experts()
        E, H, I = 256, 7168, 2048
        layer = torch.nn.Module()
        layer.moe_config = types.SimpleNamespace(experts_per_token=8, has_bias=False)
        layer.renormalize, layer.scoring_func, layer.e_score_correction_bias = True, "sigmoid", bias
        layer.use_grouped_topk, layer.num_expert_group, layer.topk_group = True, 8, 4
        layer.routed_scaling_factor, layer.custom_routing_function, layer.activation = 2.5, None, "silu"
        saved = {v: os.environ.pop(v, None) for v in ("MOE_REQUANTIZE_WEIGHT_DTYPE", "MOE_REQUANTIZE_BLOCK_SIZE",
                                                      "QMOE_FP8_NATIVE_BLOCKS")}
        try:
            if qd == "int8":
                os.environ["MOE_REQUANTIZE_WEIGHT_DTYPE"] = "int8"
            method = q.Fp8MoEMethod(q.Fp8Config(weight_block_size=[128, 128]), layer.moe_config)
            method.create_weights(layer, E, H, I, torch.bfloat16)
            layer.w13_weight.data, layer.w2_weight.data = w13, w2
            layer.w13_weight_scale_inv.data, layer.w2_weight_scale_inv.data = s13, s2
            method.process_weights_after_loading(layer)
        finally:
            for v, val in saved.items():
                os.environ.pop(v, None)
                if val is not None:
                    os.environ[v] = val
        assert layer._qmoe_format == qd
        # the requantized codes and scales of a few experts, bit-exact
        for e in (0, 131, 255):
            for wt, st, c, sc in ((w13, s13, layer.w13_weight, layer.w13_weight_scale),
                                  (w2, s2, layer.w2_weight, layer.w2_weight_scale)):
                rq, rs = quant.quantize_tensor(quant.dequant_tiles(_np(wt[e].view(torch.uint8)), _np(st[e])), qd)
                np.testing.assert_array_equal(_np(c[e].view(torch.uint8)), rq.view(np.uint8))
                np.testing.assert_array_equal(_np(sc[e]).reshape(rs.shape), rs)
        # the shared expert as a default dense FP8 linear: the same tiles
        # dequantized and requantized per channel (`fp8.py:297-348`)
        from qmoe import ops
        from qmoe.layers.quantization.fp8 import dequantize_fp8_weight

        _, _, _, _, sh13, ss13, sh2, ss2, _ = _cfg4_experts()
        shared = []
        for wt, st in ((sh13, ss13), (sh2, ss2)):
            qc, sc = ops.row_quant(dequantize_fp8_weight(wt, weight_scale_inv=st, block=(128, 128)), qd, mode="load")
            rq, rs = quant.quantize_tensor(quant.dequant_tiles(_np(wt.view(torch.uint8)), _np(st)), qd)
            np.testing.assert_array_equal(_np(qc.view(torch.uint8)), rq.view(np.uint8))
            np.testing.assert_array_equal(_np(sc), rs)
            shared += [qc, sc]
        _E4D.update(qd=qd, layer=layer, method=method, shared=shared)
    return _E4D["method"], _E4D["layer"]


@pytest.mark.parametrize("T", [1, 8, 64, 512, 4096])
@pytest.mark.parametrize("qd", ["fp8", "int8"])
def test_cfg4_default_recipe(dev, qd, T):
    """Config 4 through the method's DEFAULT recipe -- what a DeepSeek-V3
    checkpoint loaded by `Fp8MoEMethod` runs without this build's opt-in
    native tiles: per-channel e4m3 (or int8) experts and per-(token, 512)
    bf16-arithmetic activation codes before each grouped GEMM
    (`kernels/megablox/gmm_v2.py:500-548, 1198-1237`). Ids of every token
    bit-exact; the layer output on a token sample against the oracle's
    grouped-matmul recipe."""
    from qmoe import ops

    E, k, H = 256, 8, 7168
    print(f"cfg4 default recipe {qd} T={T}", flush=True)
    method, layer = _cfg4_default_layer(qd)
    bias = layer.e_score_correction_bias
    g = _gen(530 + T)
    x = torch.randn((T, H), device="cuda", generator=g).to(torch.bfloat16)
    logits = _cfg4_logits(T, False, g)
    y = _run(lambda: method.apply_monolithic(layer, x, logits))
    tw, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5,
                            num_expert_group=8, topk_group=4)
    _, ids_ref = routing.grouped_topk(_np(logits.float()), k, True, 8, 4, "sigmoid", _np(bias), 2.5)
    np.testing.assert_array_equal(_np(ids), ids_ref)
    toks = _rows_sample(T, 3)
    codes = (lambda t: t.view(torch.uint8)) if qd == "fp8" else (lambda t: t)
    ew = omoe.ExpertWeights(qd, _DeviceExperts(codes(layer.w13_weight)),
                            _DeviceExperts(layer.w13_weight_scale.reshape(E, -1)),
                            _DeviceExperts(codes(layer.w2_weight)),
                            _DeviceExperts(layer.w2_weight_scale.reshape(E, -1)), keep=False)
    ref = omoe.fused_moe_tokens(_np(x[toks].float()), ew, _np(tw[toks].float()), ids_ref[toks], "silu", E)
    assert_close_rows(_np(y[toks].float()), ref, f"cfg4 default {qd} T={T}")

    # the shared expert beside it: per-token activation codes, silu fused
    # into the gate_up GEMM, the intermediate re-quantized per token
    from qmoe import _capi

    qs13, cs13, qs2, cs2 = _E4D["shared"]
    wf, I = (0 if qd == "fp8" else 1), 2048

    def shared():
        xq, xs = ops.row_quant(x, qd)
        a = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), qs13.view(torch.uint8), a_scale=xs, w_scale=cs13,
                     wfmt=wf, activation="silu")
        aq, as_ = ops.row_quant(a, qd)
        return a, ops.gemm(_capi.W8A8_PC, aq.view(torch.uint8), qs2.view(torch.uint8), a_scale=as_, w_scale=cs2,
                           wfmt=wf)

    a, ys = _run(shared)
    toks = _rows_sample(T, 8)
    q13n = _np(qs13.view(torch.uint8)) if qd == "fp8" else _np(qs13)
    gu, _, _ = linear.w8a8_per_channel(_np(x[toks].float()), q13n, _np(cs13), qd)
    assert_close_rows(_np(a[toks].float()), codecs.bf16_round(omoe.act_fn(gu[:, :I], gu[:, I:], "silu")),
                      f"cfg4 default shared gate_up {qd} T={T}")
    q2n = _np(qs2.view(torch.uint8)) if qd == "fp8" else _np(qs2)
    ref2, _, _ = linear.w8a8_per_channel(_np(a[toks].float()), q2n, _np(cs2), qd)
    if qd == "int8":
        np.testing.assert_array_equal(_np(ys[toks].float()), ref2)
    else:
        assert_close_same_codes(_np(ys[toks].float()), ref2, f"cfg4 default shared down {qd} T={T}")


def test_cfg4_default_recipe_release():
    """Frees the processed default-recipe layer (11.3 GB) before the
    module's later tests."""
    _E4D.clear()
    torch.cuda.empty_cache()


# ------------------------------------------------------------------ coverage


def _bench_plans():
    """The kernel plans of every GEMM of bench.py's config points (configs
    0-4), computed on the host from their shapes."""
    from qmoe import _capi, ops

    plans = {}
    for M in (1, 16, 128):
        plans[f"cfg0 M={M}"] = [ops.plan_for_shape(_capi.W4A16_MX, M, 5760, 2880)]
    for wf in (0, 1):
        for K, N in ((4096, 14336), (14336, 4096)):
            for M in (1, 8, 64, 512, 4096):
                plans[f"cfg1 wfmt={wf} M={M} K={K}"] = [ops.plan_for_shape(_capi.W8A8_PC_DYN, M, N, K, wfmt=wf)]
    for N in (18432, 24576):
        for M in (1, 32, 256, 2048, 8192):
            plans[f"cfg2 M={M} N={N}"] = [ops.plan_for_shape(_capi.W8A8_BLK, M, N, 7168, ws_bn=128)]
    for T in (1, 16, 128, 1024, 8192):
        plans[f"cfg3 T={T}"] = [
            ops.plan_for_shape(_capi.W4A16_MX, 4 * T, 5760, 2880, activation="swigluoai", experts=128, max_rows=T),
            ops.plan_for_shape(_capi.W4A16_MX, 4 * T, 2880, 2880, experts=128, max_rows=T)]
    for T in (1, 8, 64, 512, 4096):
        plans[f"cfg4 T={T}"] = [
            ops.plan_for_shape(_capi.W8A8_BLK, 8 * T, 4096, 7168, activation="silu", experts=256, max_rows=T,
                               ws_bn=128),
            ops.plan_for_shape(_capi.W8A8_BLK, 8 * T, 7168, 2048, experts=256, max_rows=T, ws_bn=128),
            ops.plan_for_shape(_capi.W8A8_BLK, T, 4096, 7168, activation="silu", ws_bn=128),
            ops.plan_for_shape(_capi.W8A8_BLK, T, 7168, 2048, ws_bn=128)]
    for wf in (0, 1):
        for T in (1, 8, 64, 512, 4096):
            plans[f"cfg4 default wfmt={wf} T={T}"] = [
                ops.plan_for_shape(_capi.W8A8_GMM, 8 * T, 4096, 7168, wfmt=wf, activation="silu", experts=256,
                                   max_rows=T),
                ops.plan_for_shape(_capi.W8A8_GMM, 8 * T, 7168, 2048, wfmt=wf, experts=256, max_rows=T),
                ops.plan_for_shape(_capi.W8A8_PC, T, 4096, 7168, wfmt=wf, activation="silu"),
                ops.plan_for_shape(_capi.W8A8_PC, T, 7168, 2048, wfmt=wf)]
    return plans


def test_zz_bench_plans_are_parity_checked(dev):
    """Every (kernel, tile, K split) that a benchmark config point runs was
    run by a parity test above (needs the whole module in this session)."""
    if not _PLANS:
        pytest.skip("run together with the config tests of this module")
    missing = {name: [p for p in ps if p not in _PLANS] for name, ps in _bench_plans().items()}
    missing = {k: v for k, v in missing.items() if v}
    assert not missing, f"benchmark plans without a parity test: {missing}"
