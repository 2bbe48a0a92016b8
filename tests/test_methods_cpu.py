"""Host-side behaviour of the quant-method layer (no GPU): env-gate
validation with the reference's error texts (`fp8.py:241-259`), method
dispatch, and the checkpoint parameter shapes `create_weights` registers."""

import types

import pytest
import torch

from qmoe.layers import quantization as q


def _moe_layer(**kw):
    layer = torch.nn.Module()
    layer.moe_config = types.SimpleNamespace(experts_per_token=kw.get("k", 2), has_bias=True)
    return layer


def test_blockwise_kernel_requires_block_size(monkeypatch):
    monkeypatch.setenv("ENABLE_QUANTIZED_MATMUL_KERNEL", "1")
    monkeypatch.delenv("REQUANTIZE_BLOCK_SIZE", raising=False)
    with pytest.raises(ValueError, match="REQUANTIZE_BLOCK_SIZE"):
        q.Fp8LinearMethod(q.Fp8Config())


def test_block_size_requires_blockwise_kernel(monkeypatch):
    monkeypatch.delenv("ENABLE_QUANTIZED_MATMUL_KERNEL", raising=False)
    monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "128")
    with pytest.raises(ValueError, match="Blockwise quantization is supported by quantized matmul kernel"):
        q.Fp8LinearMethod(q.Fp8Config())


def test_unsupported_requant_dtype(monkeypatch):
    monkeypatch.setenv("REQUANTIZE_WEIGHT_DTYPE", "float8_e5m2fnuz")
    with pytest.raises(ValueError, match="Unsupported REQUANTIZE_WEIGHT_DTYPE"):
        q.Fp8LinearMethod(q.Fp8Config())


def test_e5m2_requant_dtype(monkeypatch):
    """float8_e5m2 is a requantization target of both env gates
    (`fp8.py:122-127`); the 128-column block regime stays e4m3-only."""
    from qmoe.layers.fused_moe import infer_weight_format
    from qmoe.layers.quantization import fp8

    for v in ("ENABLE_QUANTIZED_MATMUL_KERNEL", "REQUANTIZE_BLOCK_SIZE", "MOE_REQUANTIZE_BLOCK_SIZE"):
        monkeypatch.delenv(v, raising=False)
    monkeypatch.setenv("REQUANTIZE_WEIGHT_DTYPE", "float8_e5m2")
    monkeypatch.setenv("MOE_REQUANTIZE_WEIGHT_DTYPE", "float8_e5m2")
    assert fp8.get_linear_quant_config()[:3] == ("float8_e5m2", torch.float8_e5m2, None)
    assert fp8.get_moe_quant_config() == ("float8_e5m2", torch.float8_e5m2, None)
    monkeypatch.setenv("ENABLE_QUANTIZED_MATMUL_KERNEL", "1")
    monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "512")
    assert fp8.get_linear_quant_config()[2] == 512
    monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "128")
    with pytest.raises(NotImplementedError, match="float8_e4m3fn"):
        fp8.get_linear_quant_config()
    monkeypatch.setenv("MOE_REQUANTIZE_BLOCK_SIZE", "128")
    with pytest.raises(NotImplementedError, match="float8_e4m3fn"):
        fp8.get_moe_quant_config()
    w = torch.zeros((2, 4, 8), dtype=torch.float8_e5m2)
    assert infer_weight_format(w, torch.ones((2, 4))) == "e5m2"


def test_negative_w8a16_rows_rejected(monkeypatch):
    monkeypatch.setenv("TPU_FP8_LINEAR_W8A16_MAX_ROWS", "-1")
    with pytest.raises(ValueError):
        q.Fp8LinearMethod(q.Fp8Config())


def test_config_dispatch():
    cfg = q.Fp8Config.from_config({"quant_method": "fp8", "weight_block_size": [128, 128]})
    assert cfg.is_checkpoint_fp8_serialized and cfg.weight_block_size == [128, 128]
    assert isinstance(cfg.get_quant_method(torch.nn.Module()), q.Fp8LinearMethod)
    assert isinstance(cfg.get_quant_method(_moe_layer()), q.Fp8MoEMethod)
    m = q.Mxfp4Config()
    assert isinstance(m.get_quant_method(torch.nn.Module()), q.UnquantizedLinearMethod)
    assert isinstance(m.get_quant_method(_moe_layer()), q.Mxfp4MoEMethod)
    assert q.get_quantization_config("fp8") is q.Fp8Config
    with pytest.raises(ValueError):
        q.get_quantization_config("gptq")
    with pytest.raises(ValueError):
        q.Fp8Config(activation_scheme="static")


def test_fp8_create_weights_shapes():
    cfg = q.Fp8Config(weight_block_size=[128, 128])
    layer = torch.nn.Module()
    q.Fp8LinearMethod(cfg).create_weights(layer, 512, [256, 128], 512, 384, torch.bfloat16)
    assert layer.weight.shape == (384, 512) and layer.weight.dtype == torch.float8_e4m3fn
    assert layer.weight_scale_inv.shape == (3, 4)
    moe = _moe_layer()
    q.Fp8MoEMethod(cfg).create_weights(moe, 4, 256, 384, torch.bfloat16)
    assert moe.w13_weight.shape == (4, 768, 256) and moe.w2_weight.shape == (4, 256, 384)
    assert moe.w13_weight_scale_inv.shape == (4, 6, 2) and moe.w2_weight_scale_inv.shape == (4, 2, 3)


def test_mxfp4_create_weights_shapes():
    moe = _moe_layer()
    q.Mxfp4MoEMethod().create_weights(moe, 8, 2880, 2880, torch.bfloat16)
    assert moe.w13_weight.shape == (8, 5760, 1440) and moe.w13_weight.dtype == torch.uint8
    assert moe.w13_weight_scale.shape == (8, 5760, 90)
    assert moe.w2_weight.shape == (8, 2880, 1440) and moe.w2_weight_scale.shape == (8, 2880, 90)
    assert moe.w13_bias.shape == (8, 5760) and moe.w2_bias.shape == (8, 2880)
    with pytest.raises(ValueError):
        q.Mxfp4MoEMethod().create_weights(_moe_layer(), 8, 2880, 2890, torch.bfloat16)


def test_activation_codes():
    from qmoe import ops

    assert ops.act_code("gelu") == ops.act_code("gelu_tanh")  # jax.nn.gelu is approximate
    assert ops.act_code("situ:2.0:none")[2] < 0
    with pytest.raises(NotImplementedError):
        ops.act_code("relu")


def test_nvfp4_config_dispatch_and_shapes():
    """ModelOpt NVFP4 (`nvfp4.py:236-297`): linear and MoE methods, excluded
    modules run unquantized; the checkpoint parameters upstream registers."""
    cfg = q.Nvfp4Config.from_config({"quantization": {"quant_algo": "NVFP4", "group_size": 16,
                                                      "exclude_modules": ["lm_head"]}})
    assert q.get_quantization_config("modelopt_fp4") is q.Nvfp4Config and cfg.get_name() == "modelopt_fp4"
    assert isinstance(cfg.get_quant_method(torch.nn.Module(), "model.layers.0.mlp"), q.Nvfp4LinearMethod)
    assert isinstance(cfg.get_quant_method(_moe_layer(), "model.layers.0.mlp.experts"), q.Nvfp4MoEMethod)
    assert isinstance(cfg.get_quant_method(torch.nn.Module(), "lm_head"), q.UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(_moe_layer(), "lm_head"), q.UnquantizedFusedMoEMethod)
    with pytest.raises(ValueError):
        q.Nvfp4Config(group_size=32)
    layer = torch.nn.Module()
    q.Nvfp4LinearMethod(cfg).create_weights(layer, 1024, [256, 128], 1024, 384, torch.bfloat16)
    assert layer.weight.shape == (384, 512) and layer.weight.dtype == torch.uint8
    assert layer.weight_scale.shape == (384, 64) and layer.weight_scale.dtype == torch.float8_e4m3fn
    assert layer.weight_scale_2.shape == (2,) and layer.input_scale.shape == (2,)
    moe = _moe_layer()
    q.Nvfp4MoEMethod(cfg, moe.moe_config).create_weights(moe, 4, 256, 384, torch.bfloat16)
    assert moe.w13_weight.shape == (4, 768, 128) and moe.w13_weight_scale.shape == (4, 768, 16)
    assert moe.w2_weight.shape == (4, 256, 192) and moe.w2_weight_scale.shape == (4, 256, 24)
    assert moe.w13_weight_scale_2.shape == (4, 2) and moe.w2_weight_scale_2.shape == (4,)


def test_nvfp4_load_time_guards(monkeypatch):
    """The reference's NVFP4 load-time errors (`nvfp4.py:378-392, 695-699`),
    raised before any device work."""
    cfg = q.Nvfp4Config()
    lin = q.Nvfp4LinearMethod(cfg)
    layer = torch.nn.Module()
    lin.create_weights(layer, 64, [32, 32], 64, 64, torch.bfloat16)
    layer.weight_scale_2.data = torch.tensor([1.0, 2.0])
    with pytest.raises(AssertionError, match="Fused NVFP4 projections must share one global scale"):
        lin.process_weights_after_loading(layer)

    def moe_method(act="silu", has_bias=False, gated=True):
        moe = _moe_layer()
        moe.moe_config.has_bias = has_bias
        moe.moe_config.is_act_and_mul = gated
        moe.activation = act
        return q.Nvfp4MoEMethod(cfg, moe.moe_config), moe

    m, moe = moe_method(has_bias=True)
    with pytest.raises(AssertionError, match="does not support bias"):
        m.process_weights_after_loading(moe)
    m, moe = moe_method(gated=False)
    with pytest.raises(AssertionError, match="act_and_mul"):
        m.process_weights_after_loading(moe)
    m, moe = moe_method(act="swigluoai")
    with pytest.raises(NotImplementedError, match="swigluoai"):
        m.process_weights_after_loading(moe)
    monkeypatch.setenv("MOE_REQUANTIZE_BLOCK_SIZE", "32")
    m, moe = moe_method()
    with pytest.raises(NotImplementedError, match="MOE_REQUANTIZE_BLOCK_SIZE"):
        m.process_weights_after_loading(moe)


def test_compressed_tensors_int4_dispatch_shapes_and_guards(monkeypatch):
    """Compressed-tensors packed-INT4 W4A16 MoE: checkpoint parameter shapes
    (`compressed_tensors_moe_w4a16.py:172-260`) and the reference's scheme
    errors (`:142-170`), raised before any device work."""
    def cfg(**w):
        args = {"num_bits": 4, "type": "int", "symmetric": True, "strategy": "group", "group_size": 32}
        args.update(w)
        return q.CompressedTensorsConfig.from_config({"config_groups": {"g": {"weights": args}},
                                                      "ignore": ["lm_head"]})

    assert q.get_quantization_config("compressed-tensors") is q.CompressedTensorsConfig
    m = cfg().get_quant_method(_moe_layer(), "model.layers.0.mlp.experts")
    assert isinstance(m, q.CompressedTensorsW4A16MoEMethod) and m.packed_factor == 8
    assert isinstance(cfg().get_quant_method(torch.nn.Module(), "lm_head"), q.UnquantizedLinearMethod)
    with pytest.raises(NotImplementedError):
        cfg().get_quant_method(torch.nn.Module(), "model.layers.0.self_attn.q_proj")
    moe = _moe_layer()
    m.create_weights(moe, 4, 256, 128, torch.bfloat16)
    assert moe.w13_weight_packed.shape == (4, 256, 32) and moe.w13_weight_packed.dtype == torch.int32
    assert moe.w2_weight_packed.shape == (4, 256, 16)
    assert moe.w13_weight_scale.shape == (4, 256, 8) and moe.w2_weight_scale.shape == (4, 256, 4)
    with pytest.raises(NotImplementedError, match="integer INT4 weights only"):
        q.CompressedTensorsW4A16MoEMethod({"num_bits": 4, "type": "float", "symmetric": True, "strategy": "group",
                                           "group_size": 32}).create_weights(_moe_layer(), 4, 256, 128,
                                                                             torch.bfloat16)
    # a float 4-bit group-32 scheme is MXFP4 and dispatches to its own method
    assert isinstance(cfg(type="float").get_quant_method(_moe_layer()), q.CompressedTensorsW4ANMxfp4MoEMethod)
    with pytest.raises(NotImplementedError, match="symmetric INT4 only"):
        cfg(symmetric=False).get_quant_method(_moe_layer()).create_weights(_moe_layer(), 4, 256, 128,
                                                                           torch.bfloat16)
    with pytest.raises(ValueError, match="must be divisible by group_size"):
        cfg().get_quant_method(_moe_layer()).create_weights(_moe_layer(), 4, 256, 144, torch.bfloat16)
    with pytest.raises(NotImplementedError, match="channel"):
        cfg(strategy="channel").get_quant_method(_moe_layer()).create_weights(_moe_layer(), 4, 256, 128,
                                                                              torch.bfloat16)
    bad = _moe_layer()
    m.create_weights(bad, 4, 256, 128, torch.bfloat16)
    bad.w13_weight_packed = torch.nn.Parameter(torch.empty(4, 256, 128, dtype=torch.uint8), requires_grad=False)
    with pytest.raises(NotImplementedError, match="packed in INT32"):
        m.process_weights_after_loading(bad)
    monkeypatch.setenv("MOE_REQUANTIZE_WEIGHT_DTYPE", "fp4")
    with pytest.raises(NotImplementedError, match="MOE_REQUANTIZE"):
        m.process_weights_after_loading(moe)


def _ct_cfg(weights, input_activations=None):
    return q.CompressedTensorsConfig.from_config({"config_groups": {"group_0": {
        "weights": weights, "input_activations": input_activations, "targets": ["Linear"]}}, "ignore": ["lm_head"]})


def test_compressed_tensors_dispatch():
    """`compressed_tensors.py:200-254`, `compressed_tensors_moe.py:80-116`:
    FP8 linears through the FP8 method (block / channel strategies), MoE by
    weight scheme, ignored layers unquantized, other schemes refused."""
    fp8_block = _ct_cfg({"num_bits": 8, "type": "float", "strategy": "block", "block_structure": [128, 128],
                         "dynamic": False}, {"num_bits": 8, "type": "float", "strategy": "token", "dynamic": True})
    m = fp8_block.get_quant_method(torch.nn.Module(), prefix="model.layers.0.mlp.down_proj")
    assert isinstance(m, q.Fp8LinearMethod) and m.weight_block_size == [128, 128]
    assert isinstance(fp8_block.get_quant_method(_moe_layer(), prefix="model.layers.0.mlp.experts"), q.Fp8MoEMethod)
    assert isinstance(fp8_block.get_quant_method(torch.nn.Module(), prefix="lm_head"), q.UnquantizedLinearMethod)
    fp8_ch = _ct_cfg({"num_bits": 8, "type": "float", "strategy": "channel", "dynamic": False})
    m = fp8_ch.get_quant_method(torch.nn.Module(), prefix="x")
    assert isinstance(m, q.Fp8LinearMethod) and m.quant_config.is_channel_quant and m.weight_block_size is None
    layer = torch.nn.Module()
    m.create_weights(layer, 64, [32, 32], 64, 64, torch.bfloat16)
    assert tuple(layer.weight_scale.shape) == (64, 1)
    mx = _ct_cfg({"num_bits": 4, "type": "float", "strategy": "group", "group_size": 32})
    assert isinstance(mx.get_quant_method(_moe_layer(), prefix="e"), q.CompressedTensorsW4ANMxfp4MoEMethod)
    i4 = _ct_cfg({"num_bits": 4, "type": "int", "strategy": "group", "group_size": 128})
    assert isinstance(i4.get_quant_method(_moe_layer(), prefix="e"), q.CompressedTensorsW4A16MoEMethod)
    with pytest.raises(NotImplementedError):
        i4.get_quant_method(torch.nn.Module(), prefix="x")  # dense INT4: not ported (as in the reference)
    with pytest.raises(RuntimeError, match="Unsupported TPU FusedMoe scheme"):
        _ct_cfg({"num_bits": 8, "type": "int", "strategy": "channel"}).get_quant_method(_moe_layer(), prefix="e")


def test_compressed_tensors_mxfp4_moe_weight_shapes():
    layer = _moe_layer()
    m = q.CompressedTensorsW4ANMxfp4MoEMethod(layer.moe_config)
    m.create_weights(layer, 4, 256, 128, torch.bfloat16)
    assert tuple(layer.w13_weight_packed.shape) == (4, 256, 128) and layer.w13_weight_packed.dtype == torch.uint8
    assert tuple(layer.w13_weight_scale.shape) == (4, 256, 8)
    assert tuple(layer.w2_weight_packed.shape) == (4, 256, 64) and tuple(layer.w2_weight_scale.shape) == (4, 256, 4)


def test_layout_markers():
    from qmoe.layers import linear_common as lc

    assert lc.KEEP_VLLM_LAYOUT_ATTR == "_tpu_keep_vllm_weight_layout"
    assert lc.WEIGHT_FLIPPED_ATTR == "_tpu_weight_flipped"


@pytest.mark.parametrize("experts_start", [torch.tensor(0, dtype=torch.int32), torch.tensor(8, dtype=torch.int32), 8])
def test_fused_moe_gmm_refuses_expert_parallel_offsets(experts_start):
    """The reference passes experts_start as a 0-d int32 tensor exactly when
    expert parallelism is on (`layers/adapter/fused_moe.py:241-293`); this
    build holds the whole expert set, so any tensor and any non-zero offset
    raises before anything runs (CPU tensors: no kernel is reached)."""
    from qmoe.layers.fused_moe import fused_moe_gmm

    E, H, I, T = 4, 256, 128, 3
    x = torch.zeros((T, H), dtype=torch.bfloat16)
    w1 = torch.zeros((E, 2 * I, H), dtype=torch.bfloat16)
    w2 = torch.zeros((E, H, I), dtype=torch.bfloat16)
    tw = torch.ones((T, 2), dtype=torch.float32)
    ti = torch.zeros((T, 2), dtype=torch.int32)
    with pytest.raises(NotImplementedError, match="expert parallelism"):
        fused_moe_gmm(x, w1, w2, None, None, None, None, tw, ti, experts_start, 2, "silu")


def test_mx_activation_host_logic():
    """Host side of the opt-in MX activations: the K the MX kernel takes, the
    zero padding of the weight, and the kernel route (no GPU needed)."""
    from qmoe import _capi, ops
    from qmoe.layers.linear_common import mx_padded_k, pad_mxfp4_for_mx

    assert [mx_padded_k(k) for k in (32, 1024, 2880, 3072, 4096, 7168)] == [1024, 1024, 3072, 3072, 4096, 7168]
    wq = torch.randint(0, 256, (8, 1440), dtype=torch.uint8)
    ws = torch.randint(100, 140, (8, 90), dtype=torch.uint8)
    wp, wsp = pad_mxfp4_for_mx(wq, ws)
    assert wp.shape == (8, 1536) and wsp.shape == (8, 96)
    assert torch.equal(wp[:, :1440], wq) and (wp[:, 1440:] == 0).all()
    assert torch.equal(wsp[:, :90], ws) and (wsp[:, 90:] == 127).all()
    assert ops.plan_for_shape(_capi.W4A4_MX, 8192, 5760, 3072)[4] == "tiled_mx_persistent"
    assert ops.plan_for_shape(_capi.W4A4_MX, 1, 256, 1024)[4] == "tiled_mx_persistent"
    for k in (2880, 512):  # not a multiple of 512 / fewer than 4 stages
        with pytest.raises(RuntimeError):
            ops.plan_for_shape(_capi.W4A4_MX, 256, 256, k)
    with pytest.raises(RuntimeError):  # no fused activation on the MX kernel
        ops.plan_for_shape(_capi.W4A4_MX, 256, 512, 1024, activation="silu")


def _dense_expert_args(m=16, h=512, i=512, e=4):
    x = torch.zeros((m, h), dtype=torch.bfloat16)
    w1 = torch.zeros((e, 2 * i, h), dtype=torch.float8_e4m3fn)
    w2 = torch.zeros((e, h, i), dtype=torch.float8_e4m3fn)
    s1 = torch.ones((e, 2 * i), dtype=torch.float32)
    s2 = torch.ones((e, h), dtype=torch.float32)
    return x, w1, w2, s1, s2


@pytest.mark.parametrize("unsupported", ["none", "unaligned_tokens", "bias", "activation", "scale",
                                         "bf16_weights", "unaligned_hidden", "unaligned_inter", "block_scale"])
def test_dense_expert_admission(unsupported):
    """`tests/kernels/experimental/test_moe_dense_expert.py:122-149`: the
    unsupported inputs keep the grouped path (the admission rule of
    `moe_dense_expert.py:50-90`)."""
    from qmoe.layers.fused_moe import can_use_dense_expert

    x, w1, w2, s1, s2 = _dense_expert_args()
    b1, act, fmt = None, "silu", "fp8"
    if unsupported == "unaligned_tokens":
        x = x[:15]
    elif unsupported == "bias":
        b1 = torch.zeros((w1.shape[0], 1, w1.shape[1]))
    elif unsupported == "activation":
        act = "gelu"
    elif unsupported == "scale":
        s1 = None
    elif unsupported == "bf16_weights":
        w1, fmt = w1.to(torch.bfloat16), "bf16"
    elif unsupported == "unaligned_hidden":
        x, w1, w2, s1, s2 = _dense_expert_args(h=384)
    elif unsupported == "unaligned_inter":
        x, w1, w2, s1, s2 = _dense_expert_args(i=320)
    elif unsupported == "block_scale":
        s1, fmt = torch.ones((4, 1024, 4)), "fp8_w8a16"
    assert can_use_dense_expert(x, w1, w2, s1, s2, b1, None, act, fmt) == (unsupported == "none")


def test_dense_expert_threshold_env(monkeypatch):
    """`TPU_MOE_DENSE_EXPERT_THRESHOLD` (`envs.py:642`, non-negative, 0 =
    off) counts tokens: admitted exactly when 0 < T <= threshold."""
    from qmoe import envs
    from qmoe.layers.fused_moe import _dense_expert_admitted

    x, w1, w2, s1, s2 = _dense_expert_args(m=32)
    monkeypatch.delenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", raising=False)
    assert envs.TPU_MOE_DENSE_EXPERT_THRESHOLD == 0
    assert not _dense_expert_admitted(x, w1, w2, s1, s2, None, None, "silu", "fp8")
    monkeypatch.setenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", "31")
    assert not _dense_expert_admitted(x, w1, w2, s1, s2, None, None, "silu", "fp8")
    monkeypatch.setenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", "32")
    assert _dense_expert_admitted(x, w1, w2, s1, s2, None, None, "silu", "fp8")
    monkeypatch.setenv("TPU_MOE_DENSE_EXPERT_THRESHOLD", "-1")
    with pytest.raises(ValueError):
        envs.TPU_MOE_DENSE_EXPERT_THRESHOLD


def test_merge_repeated_routes():
    """The dense-expert coefficient table in route form: repeated ids on a
    token sum their weights (f32, route order) into the first route; later
    repeats become id -1 with weight 0; +w / -w cancel to exactly 0."""
    from qmoe.layers.fused_moe import merge_repeated_routes

    ids = torch.tensor([[0, 3, 3, 1], [2, 2, 2, -1], [5, 6, 7, 8]], dtype=torch.int32)
    w = torch.tensor([[1.0, 0.375, -0.375, 0.5], [0.25, 0.25, 0.5, 0.0], [0.1, 0.2, 0.3, 0.4]],
                     dtype=torch.bfloat16)
    mw, mi = merge_repeated_routes(w, ids)
    assert mi.tolist() == [[0, 3, -1, 1], [2, -1, -1, -1], [5, 6, 7, 8]]
    assert mw.dtype == torch.bfloat16
    assert mw[0].float().tolist() == [1.0, 0.0, 0.0, 0.5]
    assert mw[1].float().tolist() == [1.0, 0.0, 0.0, 0.0]
    assert torch.equal(mw[2], w[2])
