"""NVFP4 (ModelOpt FP4) quant config and methods (the reference's
`layers/adapter/quantization/nvfp4.py`).

A ModelOpt NVFP4 checkpoint holds e2m1 codes packed two per byte along K (low
nibble = even k), one e4m3 scale per 16 K values and a float32 per-tensor
global scale:
  linear: ``weight u8 [N, K/2]``, ``weight_scale e4m3 [N, K/16]``,
          ``weight_scale_2 f32 [partitions]`` (one value shared by the fused
          projections), ``input_scale`` (unused: W4A16);
  MoE:    ``w13_weight u8 [E, 2I, H/2]``, ``w13_weight_scale e4m3 [E, 2I, H/16]``,
          ``w13_weight_scale_2 f32 [E, 2]`` (gate rows, up rows),
          ``w2_weight u8 [E, H, I/2]``, ``w2_weight_scale e4m3 [E, H, I/16]``,
          ``w2_weight_scale_2 f32 [E]``.

`process_weights_after_loading` fuses each block scale with its global scale
in float32 (`nvfp4.py:398-409, 700-714`) and stores the product rounded to
bf16 -- the value the reference's block-16 dequantization multiplies with
(it casts the scale to the bf16 activation dtype, `kernels/megablox/
gmm_v2.py:452-462`). The codes stay resident as loaded (N-major, the
checkpoint layout); the kernels expand each weight to bf16(code * scale) in
registers and run bf16 activations (W4A16) with f32 accumulation, as the
reference does. Runtime scale layout: bf16 ``[N, K/16]`` / ``[E, N, K/16]``.
"""

import torch

from qmoe import envs
from qmoe.layers.fused_moe import moe_forward
from qmoe.layers.linear_common import quantized_matmul_fp4
from qmoe.layers.quantization.fp8 import _activation, _device, _param

FP8 = torch.float8_e4m3fn


def fuse_block_scales(block_scale, global_scale, halves=False):
    """float32 block scale x float32 global scale, rounded to bf16.

    ``halves``: MoE w13, whose [E, 2] global applies column 0 to the gate
    rows and column 1 to the up rows (`nvfp4.py:398-409`)."""
    s = block_scale.to(torch.float32)
    g = global_scale.to(s.device, torch.float32)
    if halves:
        n = s.shape[1] // 2
        s = torch.cat([s[:, :n] * g[:, 0].view(-1, 1, 1), s[:, n:] * g[:, 1].view(-1, 1, 1)], dim=1)
    elif g.dim() == 0 or g.numel() == 1:
        s = s * g.reshape(())
    else:
        s = s * g.view(-1, *([1] * (s.dim() - 1)))
    return s.to(torch.bfloat16).contiguous()


class Nvfp4Config:
    """Quant config for ModelOpt NVFP4 checkpoints (`nvfp4.py:236-297`)."""

    def __init__(self, group_size=16, exclude_modules=None):
        if group_size != 16:
            raise ValueError(f"NVFP4 checkpoints use 16-wide scale blocks, got group_size={group_size}")
        self.group_size = group_size
        self.exclude_modules = exclude_modules or []

    @classmethod
    def get_name(cls):
        return "modelopt_fp4"

    @classmethod
    def from_config(cls, config: dict):
        q = config.get("quantization", config)
        return cls(group_size=q.get("group_size", 16), exclude_modules=q.get("exclude_modules"))

    def is_layer_excluded(self, prefix):
        return any(prefix.startswith(p) for p in self.exclude_modules)

    def get_quant_method(self, layer, prefix=""):
        from qmoe.layers.quantization.unquantized import UnquantizedFusedMoEMethod, UnquantizedLinearMethod

        moe = hasattr(layer, "moe_config")
        if self.is_layer_excluded(prefix):
            return UnquantizedFusedMoEMethod(layer.moe_config) if moe else UnquantizedLinearMethod()
        return Nvfp4MoEMethod(self, layer.moe_config) if moe else Nvfp4LinearMethod(self)


class Nvfp4LinearMethod:
    """Dense NVFP4 weight x bf16 activation linear (`nvfp4.py:602-761`)."""

    def __init__(self, quant_config: Nvfp4Config):
        self.quant_config = quant_config
        self.group_size = quant_config.group_size

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        n = sum(output_partition_sizes)
        k = input_size_per_partition
        if k % 32:
            raise ValueError(f"NVFP4 input size {k} is not a multiple of 32")
        parts = len(output_partition_sizes)
        layer.logical_widths = list(output_partition_sizes)
        layer.register_parameter("weight", _param(torch.empty(n, k // 2, dtype=torch.uint8)))
        layer.register_parameter("weight_scale", _param(torch.empty(n, k // self.group_size, dtype=FP8)))
        layer.register_parameter("weight_scale_2", _param(torch.empty(parts, dtype=torch.float32)))
        layer.register_parameter("input_scale", _param(torch.full((parts,), float("nan"))))

    def process_weights_after_loading(self, layer):
        """`nvfp4.py:700-746`: one global scale for the fused projections."""
        if getattr(layer, "_qmoe_processed", False):
            return
        g = layer.weight_scale_2.data.flatten()
        if not bool((g == g[0]).all()):
            raise AssertionError("Fused NVFP4 projections must share one global scale.")
        dev = _device()
        scale = fuse_block_scales(layer.weight_scale.data.to(dev), g[0])
        for attr in ("weight_scale_2", "input_scale"):
            if hasattr(layer, attr):
                delattr(layer, attr)
        layer.weight = _param(layer.weight.data.to(dev).view(torch.uint8).contiguous())
        layer.weight_scale = _param(scale)
        layer._qmoe_processed = True

    def apply(self, layer, x, bias=None):
        """`nvfp4.py:752-761`: the FP4 matmul, then the bias."""
        out = quantized_matmul_fp4(x, layer.weight, layer.weight_scale)
        if bias is not None:
            out = out + bias
        return out


class Nvfp4MoEMethod:
    """NVFP4 fused MoE (`nvfp4.py:300-579`, W4A16 GMM path), experts resident
    as NVFP4 codes + bf16 fused block scales."""

    is_monolithic = True
    supports_internal_mk = False

    def __init__(self, quant_config: Nvfp4Config, moe_config=None):
        self.quant_config = quant_config
        self.moe = moe_config
        self.group_size = quant_config.group_size

    def maybe_roundup_sizes(self, hidden_size, intermediate_size_per_partition, *args, **kwargs):
        return hidden_size, intermediate_size_per_partition

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        if H % 32 or I % 32:
            raise ValueError(f"NVFP4 MoE sizes must be multiples of 32, got H={H}, I={I}")
        gs, u8 = self.group_size, torch.uint8
        layer.register_parameter("w13_weight", _param(torch.empty(E, 2 * I, H // 2, dtype=u8)))
        layer.register_parameter("w13_weight_scale", _param(torch.empty(E, 2 * I, H // gs, dtype=FP8)))
        layer.register_parameter("w13_weight_scale_2", _param(torch.empty(E, 2, dtype=torch.float32)))
        layer.register_parameter("w2_weight", _param(torch.empty(E, H, I // 2, dtype=u8)))
        layer.register_parameter("w2_weight_scale", _param(torch.empty(E, H, I // gs, dtype=FP8)))
        layer.register_parameter("w2_weight_scale_2", _param(torch.empty(E, dtype=torch.float32)))
        layer.register_parameter("w13_input_scale", _param(torch.empty(E, 2, dtype=torch.float32)))
        layer.register_parameter("w2_input_scale", _param(torch.empty(E, dtype=torch.float32)))

    def process_weights_after_loading(self, layer):
        """`nvfp4.py:384-509` (W4A16 GMM recipe, block 16)."""
        if getattr(layer, "_qmoe_processed", False):
            return
        if self.moe is not None and getattr(self.moe, "has_bias", False):
            raise AssertionError("TPU NVFP4 MoE does not support bias.")
        if self.moe is not None and getattr(self.moe, "is_act_and_mul", True) is False:
            raise AssertionError("TPU NVFP4 MoE expects gated (act_and_mul) experts with a "
                                 "[gate; up] w13 layout and a per-w1/w3 global scale [E, 2].")
        act = _activation(layer)
        if act == "swigluoai":
            raise NotImplementedError("NVFP4 MoE on TPU supports act_and_mul (silu/gelu) layouts; "
                                      "swigluoai (interleaved) is not implemented.")
        if envs.MOE_REQUANTIZE_BLOCK_SIZE:
            raise NotImplementedError("qmoe runs NVFP4 experts at their native 16-wide blocks; "
                                      "unset MOE_REQUANTIZE_BLOCK_SIZE")
        dev = _device()
        s13 = fuse_block_scales(layer.w13_weight_scale.data.to(dev), layer.w13_weight_scale_2.data, halves=True)
        s2 = fuse_block_scales(layer.w2_weight_scale.data.to(dev), layer.w2_weight_scale_2.data)
        for attr in ("w13_weight_scale_2", "w2_weight_scale_2", "w13_input_scale", "w2_input_scale"):
            if hasattr(layer, attr):
                delattr(layer, attr)
        layer.w13_weight = _param(layer.w13_weight.data.to(dev).view(torch.uint8).contiguous())
        layer.w2_weight = _param(layer.w2_weight.data.to(dev).view(torch.uint8).contiguous())
        layer.w13_weight_scale = _param(s13)
        layer.w2_weight_scale = _param(s2)
        layer._qmoe_activation = act
        layer._qmoe_processed = True

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """`nvfp4.py:511-579` (single-GPU GMM branch): route, then the fused
        MoE on NVFP4 experts."""
        return moe_forward(layer, x, router_logits, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale,
                           layer.w2_weight_scale, None, None, "nvfp4",
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS, input_ids=input_ids)
