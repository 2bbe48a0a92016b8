"""Unquantized (bf16) methods (the reference's
`layers/adapter/quantization/unquantized.py`: `VllmUnquantizedLinearMethod`
`:88-146`, `VllmUnquantizedFusedMoEMethod` `:233-382`), on the W16A16 kind of
the qmoe grouped GEMM (bf16 MFMA, f32 accumulation)."""

import torch

from qmoe import _capi, envs, ops
from qmoe.layers.fused_moe import moe_forward
from qmoe.layers.quantization.fp8 import _activation, _device, _param


class UnquantizedLinearMethod:
    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        n = sum(output_partition_sizes)
        layer.register_parameter("weight", _param(torch.empty(n, input_size_per_partition,
                                                              dtype=params_dtype)))

    def process_weights_after_loading(self, layer):
        layer.weight = _param(layer.weight.data.to(_device(), torch.bfloat16).contiguous())

    def apply(self, layer, x, bias=None):
        k = x.shape[-1]
        x2 = x.reshape(-1, k).to(torch.bfloat16)
        out = ops.gemm(_capi.W16A16, x2, layer.weight).reshape(*x.shape[:-1], -1)
        if bias is not None:
            out = out + bias
        return out


class UnquantizedFusedMoEMethod:
    is_monolithic = True
    supports_internal_mk = False

    def __init__(self, moe_config=None):
        self.moe = moe_config

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        layer.register_parameter("w13_weight", _param(torch.empty(E, 2 * I, H, dtype=params_dtype)))
        layer.register_parameter("w2_weight", _param(torch.empty(E, H, I, dtype=params_dtype)))

    def process_weights_after_loading(self, layer):
        if getattr(layer, "_qmoe_processed", False):
            return
        dev = _device()
        act = _activation(layer)
        w13 = layer.w13_weight.data.to(dev, torch.bfloat16)
        b13 = getattr(layer, "w13_bias", None)
        b13 = b13.data.to(dev) if b13 is not None else None
        if act == "swigluoai":  # interleaved gate/up rows -> [g | u]
            w13 = torch.cat([w13[:, 0::2], w13[:, 1::2]], dim=1)
            if b13 is not None:
                b13 = torch.cat([b13[:, 0::2], b13[:, 1::2]], dim=1)
        layer.w13_weight = _param(w13.contiguous())
        layer.w2_weight = _param(layer.w2_weight.data.to(dev, torch.bfloat16).contiguous())
        if b13 is not None:
            layer.w13_bias = _param(b13.to(torch.float32).contiguous())
        if getattr(layer, "w2_bias", None) is not None:
            layer.w2_bias = _param(layer.w2_bias.data.to(dev, torch.float32).contiguous())
        layer._qmoe_activation = act
        layer._qmoe_processed = True

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        return moe_forward(layer, x, router_logits, layer.w13_weight, layer.w2_weight, None, None,
                           getattr(layer, "w13_bias", None), getattr(layer, "w2_bias", None), "bf16",
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS, input_ids=input_ids)
