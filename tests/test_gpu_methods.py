"""GPU parity of the quant-method layer: checkpoint -> process_weights_after_loading
-> apply / apply_monolithic, against the oracle's restatement of the same
load-time transforms and forward."""

import types

import numpy as np
import pytest
import torch

from conftest import assert_close_rows
from oracle import codecs, linear, moe as omoe, quant, routing

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _fp8(a, dev):
    return _t(a, dev).view(torch.float8_e4m3fn)


def _linear_layer(method, n, k, ckpt_codes, ckpt_scale_inv, dev):
    layer = torch.nn.Module()
    method.create_weights(layer, k, [n], k, n, torch.bfloat16)
    layer.weight.data = _fp8(ckpt_codes, dev)
    layer.weight_scale_inv.data = _t(ckpt_scale_inv, dev)
    method.process_weights_after_loading(layer)
    return layer


@pytest.mark.parametrize("mode", ["per_channel", "block128", "block512", "block512_int8", "native_tiles", "int8",
                                  "e5m2", "block512_e5m2"])
@pytest.mark.parametrize("M", [6, 300])
def test_fp8_linear_from_block_checkpoint(dev, monkeypatch, mode, M):
    """Checkpoint 128x128 FP8 -> the reference's runtime form for each env
    setting (`fp8.py:216-348`): per-channel requant (default), per (row, B)
    requant with ENABLE_QUANTIZED_MATMUL_KERNEL=1 REQUANTIZE_BLOCK_SIZE=B (a
    [1, K/B, 1, N] scale; B = 128 runs bf16-dequantized weights, B = 512 the
    per-(token, 512) quantized activations), int8 and float8_e5m2 codes (per
    channel: e5m2 activations; B = 512: e4m3 activations); native tiles only
    with QMOE_FP8_NATIVE_BLOCKS=1."""
    from qmoe.layers import quantization as q

    print(f"fp8 linear method {mode} M={M}", flush=True)
    for v in ("ENABLE_QUANTIZED_MATMUL_KERNEL", "REQUANTIZE_BLOCK_SIZE", "REQUANTIZE_WEIGHT_DTYPE",
              "QMOE_FP8_NATIVE_BLOCKS"):
        monkeypatch.delenv(v, raising=False)
    if mode in ("native_tiles", "block128"):
        monkeypatch.setenv("ENABLE_QUANTIZED_MATMUL_KERNEL", "1")
        monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "128")
    if mode.startswith("block512"):
        monkeypatch.setenv("ENABLE_QUANTIZED_MATMUL_KERNEL", "1")
        monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "512")
    if mode == "native_tiles":
        monkeypatch.setenv("QMOE_FP8_NATIVE_BLOCKS", "1")
    if mode in ("int8", "block512_int8"):
        monkeypatch.setenv("REQUANTIZE_WEIGHT_DTYPE", "int8")
    if mode in ("e5m2", "block512_e5m2"):
        monkeypatch.setenv("REQUANTIZE_WEIGHT_DTYPE", "float8_e5m2")
    rng = np.random.default_rng(3)
    N, K = 384, 1024
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, s_inv = quant.quantize_fp8_tiles(w)
    method = q.Fp8LinearMethod(q.Fp8Config(weight_block_size=[128, 128]))
    layer = _linear_layer(method, N, K, codes, s_inv, dev)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    bias = codecs.bf16_round(rng.standard_normal(N).astype(np.float32))
    got = method.apply(layer, _t(x, dev, torch.bfloat16), _t(bias, dev, torch.bfloat16)).float().cpu().numpy()
    w_deq = quant.dequant_tiles(codes, s_inv)
    if mode == "native_tiles":
        np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), codes)
        ref, _, _ = linear.w8a8_blockwise(x, codes, linear.tile_scales_to_blocks(s_inv, N))
    elif mode.startswith("block"):
        B = 128 if mode == "block128" else 512
        qd = "int8" if mode.endswith("int8") else "fp8"
        wd = "e5m2" if mode.endswith("e5m2") else qd
        wq, wsb = quant.quantize_tensor(w_deq, wd, block=B)
        assert tuple(layer.weight_scale.shape) == (1, K // B, 1, N)  # `fp8.py:270-294`
        np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), wq.view(np.uint8))
        np.testing.assert_array_equal(layer.weight_scale[0, :, 0, :].t().cpu().numpy(), wsb)
        if B == 128:
            ref = linear.w8a16_blockwise(x, wq, wsb)
        else:
            ref, _, _ = linear.w8a8_gmm(x, wq, wsb, qd, wdtype=wd)
    else:
        qd = {"int8": "int8", "e5m2": "e5m2"}.get(mode, "fp8")
        wq, ws = quant.quantize_tensor(w_deq, qd)  # `fp8.py:297-348`: dequant -> requant per channel
        np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), wq.view(np.uint8))
        np.testing.assert_array_equal(layer.weight_scale.cpu().numpy(), ws)
        ref, _, _ = linear.w8a8_per_channel(x, wq, ws, qd)
    ref = codecs.bf16_round(ref + bias[None, :])
    if mode == "int8":
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_rows(got, ref, f"fp8 linear {mode}")


def test_fp8_apply_known_answer(dev):
    """`tests/layers/adapter/quantization/test_fp8.py:1208-1238`: all-ones
    weight, scale and input -> every output equals in_dim (128)."""
    from qmoe.layers import quantization as q

    method = q.Fp8LinearMethod(q.Fp8Config(weight_block_size=[128, 128]))
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(torch.ones(64, 128, device=dev).to(torch.float8_e4m3fn),
                                      requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(torch.ones(64, device=dev), requires_grad=False)
    out = method.apply(layer, torch.ones(4, 128, device=dev, dtype=torch.bfloat16))
    assert out.shape == (4, 64)
    assert torch.all(out.float() == 128.0)


def _moe_layer(k, act, renormalize=True, scoring="softmax", bias=None, grouped=None, rsf=1.0):
    layer = torch.nn.Module()
    layer.moe_config = types.SimpleNamespace(experts_per_token=k, has_bias=True)
    layer.renormalize = renormalize
    layer.scoring_func = scoring
    layer.e_score_correction_bias = bias
    layer.use_grouped_topk = grouped is not None
    layer.num_expert_group, layer.topk_group = grouped if grouped else (None, None)
    layer.routed_scaling_factor = rsf
    layer.custom_routing_function = None
    layer.activation = act
    return layer


@pytest.mark.parametrize("native", [False, True])
def test_fp8_moe_block_checkpoint_sigmoid_grouped(dev, monkeypatch, native):
    """DeepSeek-V3-form layer: 128x128 FP8 experts, sigmoid + bias, grouped
    top-k, routed_scaling_factor. By default the experts are requantized per
    channel and run the reference's per-(token, 512) recipe
    (`fp8.py:486-617`); with QMOE_FP8_NATIVE_BLOCKS=1 the native tiles stay
    resident (the blockwise W8A8 recipe of BASELINE config 4)."""
    from qmoe.layers import quantization as q

    print(f"fp8 moe method native={native}", flush=True)
    for v in ("MOE_REQUANTIZE_WEIGHT_DTYPE", "MOE_REQUANTIZE_BLOCK_SIZE", "QMOE_FP8_NATIVE_BLOCKS"):
        monkeypatch.delenv(v, raising=False)
    if native:
        monkeypatch.setenv("QMOE_FP8_NATIVE_BLOCKS", "1")
    rng = np.random.default_rng(7)
    E, H, I, k, T = 16, 256, 256, 4, 9
    cfg = q.Fp8Config(weight_block_size=[128, 128])
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    layer = _moe_layer(k, "silu", scoring="sigmoid", bias=_t(bias, dev), grouped=(4, 2), rsf=2.5)
    method = q.Fp8MoEMethod(cfg, layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    w13f = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2f = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    t13 = [quant.quantize_fp8_tiles(w13f[e]) for e in range(E)]
    t2 = [quant.quantize_fp8_tiles(w2f[e]) for e in range(E)]
    c13, s13 = np.stack([a for a, _ in t13]), np.stack([b for _, b in t13])
    c2, s2 = np.stack([a for a, _ in t2]), np.stack([b for _, b in t2])
    layer.w13_weight.data = _fp8(c13, dev)
    layer.w2_weight.data = _fp8(c2, dev)
    layer.w13_weight_scale_inv.data = _t(s13, dev)
    layer.w2_weight_scale_inv.data = _t(s2, dev)
    method.process_weights_after_loading(layer)
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.grouped_topk(logits, k, True, 4, 2, "sigmoid", bias, 2.5)
    if native:
        assert layer._qmoe_format == "fp8_block"
        ew = omoe.ExpertWeights("fp8_block", c13, s13, c2, s2)
    else:
        assert layer._qmoe_format == "fp8"
        r13 = [quant.quantize_tensor(quant.dequant_tiles(c13[e], s13[e]), "fp8") for e in range(E)]
        r2 = [quant.quantize_tensor(quant.dequant_tiles(c2[e], s2[e]), "fp8") for e in range(E)]
        ew = omoe.ExpertWeights("fp8", np.stack([a for a, _ in r13]), np.stack([b for _, b in r13]),
                                np.stack([a for a, _ in r2]), np.stack([b for _, b in r2]))
    ref, _, _ = omoe.fused_moe(x, ew, tw, ids, "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, "fp8 moe method")


@pytest.mark.parametrize("dtype,block,I,unpadded,dense", [("int8", None, 128, None, False),
                                                           ("float8_e4m3fn", 128, 256, None, False),
                                                           ("float8_e4m3fn", 512, 512, None, False),
                                                           ("float8_e4m3fn", None, 192, None, False),
                                                           ("float8_e4m3fn", None, 256, 200, False),
                                                           ("float8_e4m3fn", None, 128, None, True),
                                                           ("float8_e5m2", None, 256, None, False),
                                                           ("float8_e5m2", 512, 512, None, False)])
def test_fp8_moe_requant_switches(dev, monkeypatch, dtype, block, I, unpadded, dense):
    """MOE_REQUANTIZE_WEIGHT_DTYPE / MOE_REQUANTIZE_BLOCK_SIZE (`fp8.py:185-213`):
    int8 per channel (int8 activations per (token, 512)), fp8 per (row, 128)
    (bf16-dequantized weights) and per (row, 512), e5m2 per channel and per
    (row, 512) (e4m3 activations per (token, 512)); an intermediate size that
    is not a multiple of 128 is zero-padded to one, and the padding of an
    unpadded intermediate size is zeroed (`fp8.py:351-406, 515-522`). With
    ``dense``, a 16-token step under TPU_MOE_DENSE_EXPERT_THRESHOLD: the
    method's per-channel runtime layout is admitted to the dense-expert
    branch (`layers/core/fused_moe_gmm.py:669-686`), here on the fused
    route + dispatch route of `moe_forward`."""
    from qmoe.layers import quantization as q

    print(f"fp8 moe requant {dtype} block={block} I={I} unpadded={unpadded}", flush=True)
    for v in ("MOE_REQUANTIZE_WEIGHT_DTYPE", "MOE_REQUANTIZE_BLOCK_SIZE", "QMOE_FP8_NATIVE_BLOCKS"):
        monkeypatch.delenv(v, raising=False)
    monkeypatch.setenv("MOE_REQUANTIZE_WEIGHT_DTYPE", dtype)
    if block:
        monkeypatch.setenv("MOE_REQUANTIZE_BLOCK_SIZE", str(block))
    rng = np.random.default_rng(17 + I)
    E, H, k, T = 8, 512, 2, (16 if dense else 11)
    monkeypatch.setenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", "16" if dense else "0")
    layer = _moe_layer(k, "silu")
    if unpadded:
        layer.moe_config.intermediate_size_per_partition_unpadded = unpadded
    method = q.Fp8MoEMethod(q.Fp8Config(), layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    w13f = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2f = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    s13 = (rng.random((E, 2)) * 1e-3 + 1e-4).astype(np.float32)
    s2 = (rng.random(E) * 1e-3 + 1e-4).astype(np.float32)
    c13 = codecs.e4m3_encode(np.clip(w13f / np.repeat(s13, I, axis=1)[:, :, None], -448, 448))
    c2 = codecs.e4m3_encode(np.clip(w2f / s2[:, None, None], -448, 448))
    layer.w13_weight.data = _fp8(c13, dev)
    layer.w2_weight.data = _fp8(c2, dev)
    layer.w13_weight_scale.data = _t(s13, dev)
    layer.w2_weight_scale.data = _t(s2, dev)
    method.process_weights_after_loading(layer)
    real = unpadded or I
    Ip = (I + 127) // 128 * 128
    d13 = codecs.e4m3_decode(c13) * np.repeat(s13, I, axis=1)[:, :, None]
    d2 = codecs.e4m3_decode(c2) * s2[:, None, None]
    p13 = np.zeros((E, 2 * Ip, H), np.float32)
    p13[:, :real], p13[:, Ip:Ip + real] = d13[:, :real], d13[:, I:I + real]
    p2 = np.zeros((E, H, Ip), np.float32)
    p2[:, :, :real] = d2[:, :, :real]
    qd = {"int8": "int8", "float8_e5m2": "e5m2"}.get(dtype, "fp8")
    r13 = [quant.quantize_tensor(p13[e], qd, block=block) for e in range(E)]
    r2 = [quant.quantize_tensor(p2[e], qd, block=block) for e in range(E)]
    w13q, w13s = np.stack([a for a, _ in r13]), np.stack([b for _, b in r13])
    w2q, w2s = np.stack([a for a, _ in r2]), np.stack([b for _, b in r2])
    np.testing.assert_array_equal(layer.w13_weight.data.view(torch.uint8).cpu().numpy(), w13q.view(np.uint8))
    np.testing.assert_array_equal(layer.w2_weight_scale.cpu().numpy().reshape(w2s.shape), w2s)
    fmt = "fp8_w8a16" if block == 128 else qd
    assert layer._qmoe_format == fmt
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    if dense:
        from qmoe.layers.fused_moe import _dense_expert_admitted

        assert _dense_expert_admitted(_t(x, dev, torch.bfloat16), layer.w13_weight, layer.w2_weight,
                                      layer.w13_weight_scale, layer.w2_weight_scale, None, None, "silu", fmt)
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights(fmt, w13q, w13s, w2q, w2s), tw, ids, "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, f"fp8 moe requant {dtype} {block}")
    if dense:
        d = omoe.dense_expert_moe(x, w13q, w13s.reshape(E, -1), w2q, w2s.reshape(E, -1), tw, ids)
        g = got.float().cpu().numpy().astype(np.float64)
        assert np.sum(g * d) / (np.linalg.norm(g) * np.linalg.norm(d)) >= 0.9995


def test_mxfp4_moe_interleaved_checkpoint_swigluoai(dev):
    """GPT-OSS-form layer: MXFP4 experts with interleaved gate/up rows and
    biases, softmax top-k, swigluoai."""
    from qmoe.layers import quantization as q

    print("mxfp4 moe method", flush=True)
    rng = np.random.default_rng(11)
    E, H, I, k, T = 8, 256, 192, 2, 7
    layer = _moe_layer(k, "swigluoai")
    method = q.Mxfp4MoEMethod(layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    c13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    s13 = (127 + rng.integers(-8, 1, (E, 2 * I, H // 32))).astype(np.uint8)
    c2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    s2 = (127 + rng.integers(-8, 1, (E, H, I // 32))).astype(np.uint8)
    b13 = codecs.bf16_round((rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32))
    b2 = codecs.bf16_round((rng.standard_normal((E, H)) * 0.1).astype(np.float32))
    layer.w13_weight.data = _t(c13, dev)
    layer.w13_weight_scale.data = _t(s13, dev)
    layer.w2_weight.data = _t(c2, dev)
    layer.w2_weight_scale.data = _t(s2, dev)
    layer.w13_bias.data = _t(b13, dev, torch.bfloat16)
    layer.w2_bias.data = _t(b2, dev, torch.bfloat16)
    method.process_weights_after_loading(layer)
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    # the reference de-interleaves gate (even) / up (odd) rows at load (`mxfp4.py:257-262`)
    dei = lambda a: np.concatenate([a[:, 0::2], a[:, 1::2]], axis=1)  # noqa: E731
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("mxfp4", dei(c13), dei(s13), c2, s2, dei(b13), b2),
                               tw, ids, "swigluoai")
    assert_close_rows(got.float().cpu().numpy(), ref, "mxfp4 moe method")


@pytest.mark.parametrize("interleaved", [False, True])
def test_fp8_moe_requantized_in_expert_chunks(dev, monkeypatch, interleaved):
    """Per-expert-scale FP8 checkpoint -> the reference's default per-channel
    requantization (`fp8.py:486-617`), done on the device a few experts at a
    time (chunk limit patched down to 3 experts), with swigluoai's
    interleaved gate/up rows de-interleaved on the way; the layer output
    matches the oracle on the requantized weights."""
    from qmoe.layers import quantization as q
    from qmoe.layers.quantization import fp8 as qfp8

    print(f"fp8 moe chunked requant interleaved={interleaved}", flush=True)
    rng = np.random.default_rng(13)
    E, H, I, k, T = 8, 256, 128, 2, 5
    monkeypatch.setattr(qfp8, "REQUANT_CHUNK_BYTES", 4 * 2 * I * H * 3)
    act = "swigluoai" if interleaved else "silu"
    layer = _moe_layer(k, act)
    method = q.Fp8MoEMethod(q.Fp8Config(), layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    w13f = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2f = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    s13 = (rng.random((E, 2)) * 1e-3 + 1e-4).astype(np.float32)  # one scale per w1 / w3 shard
    s2 = (rng.random(E) * 1e-3 + 1e-4).astype(np.float32)
    c13 = codecs.e4m3_encode(np.clip(w13f / np.repeat(s13, I, axis=1)[:, :, None], -448, 448))
    c2 = codecs.e4m3_encode(np.clip(w2f / s2[:, None, None], -448, 448))
    layer.w13_weight.data = _fp8(c13, dev)
    layer.w2_weight.data = _fp8(c2, dev)
    layer.w13_weight_scale.data = _t(s13, dev)
    layer.w2_weight_scale.data = _t(s2, dev)
    method.process_weights_after_loading(layer)
    # the oracle requantizes the dequantized checkpoint per channel (load-time quantizer)
    d13 = codecs.e4m3_decode(c13) * np.repeat(s13, I, axis=1)[:, :, None]
    if interleaved:
        d13 = np.concatenate([d13[:, 0::2], d13[:, 1::2]], axis=1)
    d2 = codecs.e4m3_decode(c2) * s2[:, None, None]
    r13 = [quant.quantize_tensor(d13[e].astype(np.float32), "fp8") for e in range(E)]
    r2 = [quant.quantize_tensor(d2[e].astype(np.float32), "fp8") for e in range(E)]
    np.testing.assert_array_equal(layer.w13_weight.data.view(torch.uint8).cpu().numpy(),
                                  np.stack([a for a, _ in r13]).view(np.uint8))
    np.testing.assert_array_equal(layer.w2_weight.data.view(torch.uint8).cpu().numpy(),
                                  np.stack([a for a, _ in r2]).view(np.uint8))
    np.testing.assert_array_equal(layer.w13_weight_scale.cpu().numpy(), np.stack([b for _, b in r13]))
    np.testing.assert_array_equal(layer.w2_weight_scale.cpu().numpy(), np.stack([b for _, b in r2]))
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("fp8", np.stack([a for a, _ in r13]),
                                                      np.stack([b for _, b in r13]), np.stack([a for a, _ in r2]),
                                                      np.stack([b for _, b in r2])), tw, ids, act)
    assert_close_rows(got.float().cpu().numpy(), ref, "fp8 moe chunked requant")


def test_nvfp4_linear_from_checkpoint(dev):
    """ModelOpt NVFP4 dense linear: e2m1 codes + e4m3 block scales + a shared
    f32 global (`nvfp4.py:700-761`) -> fused bf16 block scales; apply() is the
    W4A16 matmul plus bias. The stored scales equal the oracle's fused scales
    rounded to bf16, bit for bit."""
    from qmoe.layers import quantization as q

    print("nvfp4 linear method", flush=True)
    rng = np.random.default_rng(21)
    N, K, M = 384, 1024, 5
    method = q.Nvfp4Config().get_quant_method(torch.nn.Linear(1, 1), prefix="model.layers.0.mlp")
    layer = torch.nn.Module()
    method.create_weights(layer, K, [256, 128], K, N, torch.bfloat16)
    codes = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    blk = rng.integers(0x20, 0x48, (N, K // 16)).astype(np.uint8)
    g = np.float32(0.0123456789)
    layer.weight.data = _t(codes, dev)
    layer.weight_scale.data = _fp8(blk, dev)
    layer.weight_scale_2.data = _t(np.full(2, g, np.float32), dev)
    layer.input_scale.data = _t(np.ones(2, np.float32), dev)
    method.process_weights_after_loading(layer)
    assert not hasattr(layer, "weight_scale_2") and not hasattr(layer, "input_scale")
    fused = codecs.nvfp4_fuse_scales(blk, g)
    np.testing.assert_array_equal(layer.weight_scale.float().cpu().numpy(), codecs.bf16_round(fused))
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    bias = codecs.bf16_round(rng.standard_normal(N).astype(np.float32))
    got = method.apply(layer, _t(x, dev, torch.bfloat16), _t(bias, dev, torch.bfloat16))
    ref = codecs.bf16_round(linear.w4a16_nvfp4(x, codes, fused) + bias)
    assert_close_rows(got.float().cpu().numpy(), ref, "nvfp4 linear method")


@pytest.mark.parametrize("T", [3, 150])
def test_nvfp4_moe_from_checkpoint(dev, T):
    """ModelOpt NVFP4 MoE: per-expert [gate, up] globals on w13 and a
    per-expert global on w2 (`nvfp4.py:384-509`), silu; T = 3 takes the fused
    routing + streaming path, T = 150 the tiled kernels."""
    from qmoe.layers import quantization as q

    print(f"nvfp4 moe method T={T}", flush=True)
    rng = np.random.default_rng(23 + T)
    E, H, I, k = 8, 256, 192, 2
    layer = _moe_layer(k, "silu")
    layer.moe_config.has_bias = False
    method = q.Nvfp4MoEMethod(q.Nvfp4Config(), layer.moe_config)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    c13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    c2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    b13 = rng.integers(0x20, 0x40, (E, 2 * I, H // 16)).astype(np.uint8)
    b2 = rng.integers(0x20, 0x40, (E, H, I // 16)).astype(np.uint8)
    g13 = (rng.random((E, 2)) * 0.01 + 0.003).astype(np.float32)
    g2 = (rng.random(E) * 0.01 + 0.003).astype(np.float32)
    layer.w13_weight.data = _t(c13, dev)
    layer.w2_weight.data = _t(c2, dev)
    layer.w13_weight_scale.data = _fp8(b13, dev)
    layer.w2_weight_scale.data = _fp8(b2, dev)
    layer.w13_weight_scale_2.data = _t(g13, dev)
    layer.w2_weight_scale_2.data = _t(g2, dev)
    method.process_weights_after_loading(layer)
    s13 = codecs.nvfp4_fuse_scales(b13, g13, halves=True)
    s2 = codecs.nvfp4_fuse_scales(b2, g2)
    np.testing.assert_array_equal(layer.w13_weight_scale.float().cpu().numpy(), codecs.bf16_round(s13))
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("nvfp4", c13, s13, c2, s2), tw, ids, "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, "nvfp4 moe method")


@pytest.mark.parametrize("T,group", [(4, 32), (150, 128)])
def test_compressed_tensors_int4_moe_from_checkpoint(dev, T, group):
    """Compressed-tensors packed-INT4 W4A16 MoE (`compressed_tensors_moe_w4a16.py`):
    int32 carriers + bf16 group scales as loaded, silu; T = 4 takes the fused
    routing + streaming path, T = 150 the tiled kernels."""
    from qmoe.layers import quantization as q

    print(f"ct int4 moe method T={T} group={group}", flush=True)
    rng = np.random.default_rng(31 + T)
    E, H, I, k = 8, 512, 256, 2
    layer = _moe_layer(k, "silu")
    cfg = q.CompressedTensorsConfig.from_config({"config_groups": {"group_0": {
        "weights": {"num_bits": 4, "type": "int", "symmetric": True, "strategy": "group", "group_size": group},
        "input_activations": None, "targets": ["Linear"]}}, "ignore": ["lm_head"]})
    method = cfg.get_quant_method(layer, prefix="model.layers.0.mlp.experts")
    method.create_weights(layer, E, H, I, torch.bfloat16)
    v13 = rng.integers(-8, 8, (E, 2 * I, H))
    v2 = rng.integers(-8, 8, (E, H, I))
    s13 = codecs.bf16_round((rng.random((E, 2 * I, H // group)) * 0.004 + 0.001).astype(np.float32))
    s2 = codecs.bf16_round((rng.random((E, H, I // group)) * 0.004 + 0.001).astype(np.float32))
    layer.w13_weight_packed.data = _t(codecs.int4_pack(v13), dev)
    layer.w2_weight_packed.data = _t(codecs.int4_pack(v2), dev)
    layer.w13_weight_scale.data = _t(s13, dev, torch.bfloat16)
    layer.w2_weight_scale.data = _t(s2, dev, torch.bfloat16)
    method.process_weights_after_loading(layer)
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("int4", codecs.int4_pack(v13), s13, codecs.int4_pack(v2), s2),
                               tw, ids, "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, "ct int4 moe method")
