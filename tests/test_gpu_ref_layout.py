"""The reference's runtime layouts at the op functions on the GPU: a weight
passed in the reference's K-major form (with its ``[.., K/B, 1, N]`` float32
scales) gives bit-identical outputs to the same values in this package's
N-major form (the repack moves bytes; the kernels are the same), and the
compressed-tensors MXFP4 / FP8 methods and the FP8 embedding branch against
the oracle."""

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


def _kmajor_fp4(codes_nm):
    """N-major packed codes [..., N, K/2] -> the reference's K-major packing
    [..., K, N/2] (two codes per byte along N)."""
    c = codecs.unpack_fp4(codes_nm)
    return codecs.pack_fp4(np.swapaxes(c, -1, -2).copy())


@pytest.mark.parametrize("M", [3, 200])
def test_quantized_matmul_kmajor_weight(dev, M):
    """A contiguous [n_in, n_out] weight (the reference's flipped layout)
    equals the [n_in, n_out] view of the N-major buffer."""
    from qmoe.layers.linear_common import quantized_matmul

    print(f"quantized_matmul k-major M={M}", flush=True)
    rng = np.random.default_rng(M)
    N, K = 384, 512
    wq, ws = quant.quantize_tensor((rng.standard_normal((N, K)) * 0.02).astype(np.float32), "fp8")
    x = _t(codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32)), dev, torch.bfloat16)
    w_nk = _t(wq, dev).view(torch.float8_e4m3fn)
    a = quantized_matmul(x, w_nk.t(), _t(ws, dev))
    b = quantized_matmul(x, w_nk.t().contiguous(), _t(ws, dev))
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [1, 40])
@pytest.mark.parametrize("blk", [16, 32])
def test_quantized_matmul_fp4_reference_layout(dev, M, blk):
    """K-major fp4 + [1, K/B, 1, N] float32 scale: block 16 (NVFP4, fused
    scales) and block 32 (MXFP4, power-of-two scales) equal the N-major
    forms bit for bit."""
    from qmoe.layers.linear_common import quantized_matmul_fp4

    print(f"quantized_matmul_fp4 reference layout M={M} B={blk}", flush=True)
    rng = np.random.default_rng(M + blk)
    N, K = 256, 512
    codes = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    if blk == 32:
        e8 = (127 + rng.integers(-8, 1, (N, K // 32))).astype(np.uint8)
        s_ref = codecs.e8m0_decode(e8)
        native = _t(e8, dev)
    else:
        s_ref = codecs.bf16_round((rng.random((N, K // 16)) * 0.02 + 0.001).astype(np.float32))
        native = _t(s_ref, dev, torch.bfloat16)
    x = _t(codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32)), dev, torch.bfloat16)
    a = quantized_matmul_fp4(x, _t(codes, dev), native)
    w_km = _t(_kmajor_fp4(codes), dev)
    if hasattr(torch, "float4_e2m1fn_x2"):
        w_km = w_km.view(torch.float4_e2m1fn_x2)
    b = quantized_matmul_fp4(x, w_km, _t(s_ref.T[None, :, None, :], dev))
    assert b.shape == (M, N)
    assert torch.equal(a, b)


def _moe_inputs(rng, dev, E, H, T, k):
    x = _t(codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32)), dev, torch.bfloat16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    return x, _t(tw, dev, torch.bfloat16), _t(ids, dev, torch.int32)


@pytest.mark.parametrize("fmt", ["fp8", "fp8_w8a16", "bf16", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("T", [4, 100])
def test_fused_moe_gmm_reference_layout(dev, fmt, T):
    """w1 [E, H, 2I] / w2 [E, I, H] with [E, K/B, 1, N] scales (and [E, 1, N]
    biases for the bf16 / MXFP4 forms) equal this package's [E, 2I, H] /
    [E, H, I] forms bit for bit."""
    from qmoe.layers.fused_moe import fused_moe_gmm

    print(f"fused_moe_gmm reference layout {fmt} T={T}", flush=True)
    rng = np.random.default_rng(T + len(fmt))
    E, H, I, k = 8, 512, 256, 2
    x, tw, ids = _moe_inputs(rng, dev, E, H, T, k)
    b13 = b2 = rb13 = rb2 = None
    act = "silu"
    if fmt in ("fp8", "fp8_w8a16"):
        blk = None if fmt == "fp8" else 128
        w13, s13 = quant.quantize_tensor((rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32), "fp8",
                                         block=blk)
        w2, s2 = quant.quantize_tensor((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32), "fp8", block=blk)
        n13, n2 = _t(w13, dev).view(torch.float8_e4m3fn), _t(w2, dev).view(torch.float8_e4m3fn)
        ns13, ns2 = _t(s13, dev), _t(s2, dev)
        r13, r2 = n13.transpose(1, 2).contiguous(), n2.transpose(1, 2).contiguous()
        if blk is None:
            rs13, rs2 = ns13[:, None, None, :], ns2[:, None, None, :]
        else:
            rs13, rs2 = ns13.transpose(1, 2)[:, :, None, :], ns2.transpose(1, 2)[:, :, None, :]
    elif fmt == "bf16":
        n13 = _t(rng.standard_normal((E, 2 * I, H)) * 0.02, dev, torch.bfloat16)
        n2 = _t(rng.standard_normal((E, H, I)) * 0.02, dev, torch.bfloat16)
        ns13 = ns2 = rs13 = rs2 = None
        r13, r2 = n13.transpose(1, 2).contiguous(), n2.transpose(1, 2).contiguous()
        b13 = _t(rng.standard_normal((E, 2 * I)) * 0.1, dev, torch.float32)
        b2 = _t(rng.standard_normal((E, H)) * 0.1, dev, torch.float32)
        rb13, rb2 = b13[:, None, :], b2[:, None, :]
    else:
        blk = 32 if fmt == "mxfp4" else 16
        c13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
        c2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
        if fmt == "mxfp4":
            e13 = (127 + rng.integers(-8, 1, (E, 2 * I, H // 32))).astype(np.uint8)
            e2 = (127 + rng.integers(-8, 1, (E, H, I // 32))).astype(np.uint8)
            f13, f2 = codecs.e8m0_decode(e13), codecs.e8m0_decode(e2)
            ns13, ns2 = _t(e13, dev), _t(e2, dev)
            act = "swigluoai"
            b13 = _t(codecs.bf16_round((rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32)), dev)
            b2 = _t(codecs.bf16_round((rng.standard_normal((E, H)) * 0.1).astype(np.float32)), dev)
            rb13, rb2 = b13[:, None, :], b2[:, None, :]
        else:
            f13 = codecs.bf16_round((rng.random((E, 2 * I, H // 16)) * 0.02 + 0.001).astype(np.float32))
            f2 = codecs.bf16_round((rng.random((E, H, I // 16)) * 0.02 + 0.001).astype(np.float32))
            ns13, ns2 = _t(f13, dev, torch.bfloat16), _t(f2, dev, torch.bfloat16)
        n13, n2 = _t(c13, dev), _t(c2, dev)
        r13, r2 = _t(_kmajor_fp4(c13), dev), _t(_kmajor_fp4(c2), dev)
        rs13 = _t(np.swapaxes(f13, 1, 2)[:, :, None, :], dev)
        rs2 = _t(np.swapaxes(f2, 1, 2)[:, :, None, :], dev)
    a = fused_moe_gmm(x, n13, n2, ns13, ns2, b13, b2, tw, ids, None, k, act,
                      weight_format=fmt if fmt != "fp8" else None)
    b = fused_moe_gmm(x, r13, r2, rs13, rs2, rb13, rb2, tw, ids, None, k, act)
    assert torch.equal(a, b)


def _moe_layer(k, act):
    layer = torch.nn.Module()
    layer.moe_config = types.SimpleNamespace(experts_per_token=k, has_bias=False,
                                             intermediate_size_per_partition_unpadded=None)
    layer.renormalize = True
    layer.scoring_func = "softmax"
    layer.e_score_correction_bias = None
    layer.use_grouped_topk = False
    layer.num_expert_group = layer.topk_group = None
    layer.routed_scaling_factor = 1.0
    layer.custom_routing_function = None
    layer.activation = act
    return layer


@pytest.mark.parametrize("T,mx", [(3, False), (150, False), (150, True), (2048, True)])
def test_compressed_tensors_mxfp4_moe(dev, T, mx):
    """Compressed-tensors MXFP4 MoE (`compressed_tensors_moe_w4an_mxfp4.py`):
    packed codes + e8m0 scales as loaded, silu, padded tokens skipped. With
    the opt-in MX activations (H 256 / I 192 padded to 1024): T = 150 runs
    the bf16-activation kernels on the dequantized MX activations over the
    padded weights' views, T = 2048 (512 rows per expert) the grouped MX
    tiles; against the oracle's "mxfp4_mx" recipe."""
    from qmoe.layers import quantization as q

    print(f"ct mxfp4 moe T={T} mx={mx}", flush=True)
    rng = np.random.default_rng(41 + T)
    E, H, I, k = 8, 256, 192, 2
    layer = _moe_layer(k, "silu")
    cfg = q.CompressedTensorsConfig.from_config({"config_groups": {"g": {
        "weights": {"num_bits": 4, "type": "float", "strategy": "group", "group_size": 32}}}})
    method = cfg.get_quant_method(layer, prefix="model.layers.0.mlp.experts")
    assert isinstance(method, q.CompressedTensorsW4ANMxfp4MoEMethod)
    method.mx_activations = mx
    method.create_weights(layer, E, H, I, torch.bfloat16)
    c13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
    s13 = (127 + rng.integers(-8, 1, (E, 2 * I, H // 32))).astype(np.uint8)
    c2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
    s2 = (127 + rng.integers(-8, 1, (E, H, I // 32))).astype(np.uint8)
    layer.w13_weight_packed.data = _t(c13, dev)
    layer.w13_weight_scale.data = _t(s13, dev)
    layer.w2_weight_packed.data = _t(c2, dev)
    layer.w2_weight_scale.data = _t(s2, dev)
    method.process_weights_after_loading(layer)
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("mxfp4_mx" if mx else "mxfp4", c13, s13, c2, s2), tw, ids,
                               "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, f"ct mxfp4 moe mx={mx}")


def test_compressed_tensors_fp8_channel_moe(dev):
    """Compressed-tensors FP8 MoE (channel strategy, `compressed_tensors.py:
    86-109` -> the FP8 MoE method): per-channel checkpoint scales [E, N, 1]
    dequantized and requantized per channel (the reference's default)."""
    from qmoe.layers import quantization as q

    print("ct fp8 channel moe", flush=True)
    rng = np.random.default_rng(43)
    E, H, I, k, T = 8, 256, 128, 2, 6
    layer = _moe_layer(k, "silu")
    cfg = q.CompressedTensorsConfig.from_config({"config_groups": {"g": {
        "weights": {"num_bits": 8, "type": "float", "strategy": "channel"},
        "input_activations": {"num_bits": 8, "type": "float", "strategy": "token", "dynamic": True}}}})
    method = cfg.get_quant_method(layer, prefix="e")
    assert isinstance(method, q.Fp8MoEMethod)
    method.create_weights(layer, E, H, I, torch.bfloat16)
    w13f = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
    w2f = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
    q13 = [quant.quantize_tensor(w13f[e], "fp8") for e in range(E)]
    q2 = [quant.quantize_tensor(w2f[e], "fp8") for e in range(E)]
    layer.w13_weight.data = _t(np.stack([a for a, _ in q13]), dev).view(torch.float8_e4m3fn)
    layer.w2_weight.data = _t(np.stack([a for a, _ in q2]), dev).view(torch.float8_e4m3fn)
    layer.w13_weight_scale.data = _t(np.stack([b for _, b in q13])[:, :, None], dev)
    layer.w2_weight_scale.data = _t(np.stack([b for _, b in q2])[:, :, None], dev)
    method.process_weights_after_loading(layer)
    # per-channel checkpoint -> dequantize -> requantize per channel: the oracle's
    # load-time quantizer on the dequantized rows
    d13 = np.stack([codecs.e4m3_decode(a) * b[:, None] for a, b in q13]).astype(np.float32)
    d2 = np.stack([codecs.e4m3_decode(a) * b[:, None] for a, b in q2]).astype(np.float32)
    r13 = [quant.quantize_tensor(d13[e], "fp8") for e in range(E)]
    r2 = [quant.quantize_tensor(d2[e], "fp8") for e in range(E)]
    np.testing.assert_array_equal(layer.w13_weight.data.view(torch.uint8).cpu().numpy(),
                                  np.stack([a for a, _ in r13]).view(np.uint8))
    x = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    got = method.apply_monolithic(layer, _t(x, dev, torch.bfloat16), _t(logits, dev, torch.bfloat16))
    tw, ids = routing.select_experts(logits, k, True, "softmax")
    ref, _, _ = omoe.fused_moe(x, omoe.ExpertWeights("fp8", np.stack([a for a, _ in r13]),
                                                      np.stack([b for _, b in r13]), np.stack([a for a, _ in r2]),
                                                      np.stack([b for _, b in r2])), tw, ids, "silu")
    assert_close_rows(got.float().cpu().numpy(), ref, "ct fp8 channel moe")


def test_fp8_embedding_branch(dev):
    """`fp8.py:1669-1704`: a VocabParallelEmbedding-typed layer keeps bf16
    activations in apply (W8A16 with its per-row scales), embedding() gathers
    and dequantizes rows, tie_weights shares codes and scales."""
    from qmoe.layers import quantization as q
    from qmoe.layers.linear_common import KEEP_VLLM_LAYOUT_ATTR

    print("fp8 embedding branch", flush=True)

    class VocabParallelEmbedding(torch.nn.Module):
        pass

    rng = np.random.default_rng(47)
    V, Hd = 512, 256
    method = q.Fp8LinearMethod(q.Fp8Config(is_checkpoint_fp8_serialized=False))
    emb = VocabParallelEmbedding()
    method.create_weights(emb, Hd, [V], Hd, V, torch.bfloat16)
    w = (rng.standard_normal((V, Hd)) * 0.02).astype(np.float32)
    emb.weight.data = _t(w, dev, torch.bfloat16)
    method.process_weights_after_loading(emb)
    wq, ws = emb.weight.data, emb.weight_scale.data
    assert ws.shape == (V,)
    wq_ref, ws_ref = quant.quantize_tensor(codecs.bf16_round(w), "fp8")
    np.testing.assert_array_equal(wq.view(torch.uint8).cpu().numpy(), wq_ref.view(np.uint8))
    np.testing.assert_array_equal(ws.cpu().numpy(), ws_ref)
    x = codecs.bf16_round(rng.standard_normal((5, Hd)).astype(np.float32))
    got = method.apply(emb, _t(x, dev, torch.bfloat16))
    assert_close_rows(got.float().cpu().numpy(), linear.w8a16_per_channel(x, wq_ref, ws_ref), "fp8 lm head")
    ids = torch.tensor([[3, 500], [0, 77]], device=dev)
    e = method.embedding(emb, ids)
    assert e.shape == (2, 2, Hd)
    ref = codecs.bf16_round(codecs.bf16_round(codecs.e4m3_decode(wq_ref))[[3, 500, 0, 77]]
                            * codecs.bf16_round(ws_ref[[3, 500, 0, 77]])[:, None])
    np.testing.assert_array_equal(e.float().reshape(4, Hd).cpu().numpy(), ref)
    head = torch.nn.Module()
    method.tie_weights(head, emb)
    assert head.weight is emb.weight and getattr(head, KEEP_VLLM_LAYOUT_ATTR)
