"""MXFP4 quant config and methods (the reference's
`layers/adapter/quantization/mxfp4.py` and the compressed-tensors W4A16
MXFP4 MoE method `.../compressed_tensors_moe_w4an_mxfp4.py`).

The checkpoint holds e2m1 codes packed two per byte along K (low nibble =
even k) and one e8m0 scale byte per 32 K values, N-major:
``w13_weight u8 [E, 2I, H/2]``, ``w13_weight_scale u8 [E, 2I, H/32]``,
``w2_weight u8 [E, H, I/2]``, ``w2_weight_scale u8 [E, H, I/32]`` and f32/bf16
biases ``[E, 2I]`` / ``[E, H]``. The reference's GPT-OSS method dequantizes
these to bf16 at load (`mxfp4.py:247-318`); here they stay resident as MXFP4
(the native-fp4 path of the compressed-tensors method, `:173-273`) and the
kernels expand them to bf16 in registers, exactly (a power-of-two times an
e2m1 value is exact in bf16), with bf16 activations (W4A16) as the reference
runs them. Outputs are the same; HBM traffic is 3.8x lower.

For ``swigluoai`` the checkpoint interleaves gate and up rows (gate = even
rows); they are de-interleaved once at load (`mxfp4.py:257-262`), codes,
scales and bias alike (a row permutation, exact).

Dense layers: like the reference's `Mxfp4Config.get_quant_method`
(`mxfp4.py:128-150`), linear layers of an MXFP4 checkpoint run unquantized;
`Mxfp4LinearMethod` is the native W4A16 dense path for layers whose
checkpoint weights are MXFP4.
"""

import torch

from qmoe import envs
from qmoe.layers.fused_moe import moe_forward
from qmoe.layers.linear_common import pad_mxfp4_for_mx, quantized_matmul_fp4, quantized_matmul_mxfp4_a4
from qmoe.layers.quantization.fp8 import _activation, _device, _param


class Mxfp4Config:
    """Quant config for MXFP4 checkpoints (`mxfp4.py:105-163`)."""

    def __init__(self, ignored_layers=None):
        self.ignored_layers = ignored_layers or []

    @classmethod
    def get_name(cls):
        return "mxfp4"

    @classmethod
    def from_config(cls, config: dict):
        return cls(ignored_layers=config.get("ignored_layers"))

    def get_quant_method(self, layer, prefix=""):
        from qmoe.layers.quantization.unquantized import UnquantizedLinearMethod

        if hasattr(layer, "moe_config"):
            return Mxfp4MoEMethod(layer.moe_config)
        return UnquantizedLinearMethod()


class Mxfp4LinearMethod:
    """Dense MXFP4 weight x bf16 activation linear.

    ``mx_activations`` (default: the QMOE_MXFP4_MX_ACTIVATIONS flag) opts
    into MX-quantized activations (W4A4; no counterpart in the reference):
    the weight is zero-padded along K at load to the MX kernel's multiple of
    512 (``layer.weight`` / ``layer.weight_scale`` stay views of the
    checkpoint shape) and `quantized_matmul_mxfp4_a4` runs the forward.
    """

    def __init__(self, mx_activations=None):
        self.mx_activations = envs.QMOE_MXFP4_MX_ACTIVATIONS if mx_activations is None else bool(mx_activations)

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        n = sum(output_partition_sizes)
        k = input_size_per_partition
        if k % 32:
            raise ValueError(f"MXFP4 input size {k} is not a multiple of 32")
        layer.register_parameter("weight", _param(torch.empty(n, k // 2, dtype=torch.uint8)))
        layer.register_parameter("weight_scale", _param(torch.empty(n, k // 32, dtype=torch.uint8)))

    def process_weights_after_loading(self, layer):
        dev = _device()
        layer.weight = _param(layer.weight.data.to(dev).view(torch.uint8).contiguous())
        layer.weight_scale = _param(layer.weight_scale.data.to(dev).view(torch.uint8).contiguous())
        if self.mx_activations:
            kb, ks = layer.weight.shape[1], layer.weight_scale.shape[1]
            wq, ws = pad_mxfp4_for_mx(layer.weight.data, layer.weight_scale.data)
            layer.qmoe_mx_weight, layer.qmoe_mx_weight_scale, layer.qmoe_mx_k = wq, ws, 2 * kb
            layer.weight = _param(wq[:, :kb])
            layer.weight_scale = _param(ws[:, :ks])

    def apply(self, layer, x, bias=None):
        if getattr(layer, "qmoe_mx_k", None):
            return quantized_matmul_mxfp4_a4(x, layer.qmoe_mx_weight, layer.qmoe_mx_weight_scale, layer.qmoe_mx_k,
                                             bias)
        out = quantized_matmul_fp4(x, layer.weight, layer.weight_scale)
        if bias is not None:
            out = out + bias
        return out


class Mxfp4MoEMethod:
    """MXFP4 fused MoE (`mxfp4.py:207-364`), experts resident as MXFP4.

    ``mx_activations`` (default: the QMOE_MXFP4_MX_ACTIVATIONS flag) opts
    into MX-quantized activations for both expert GEMMs (no counterpart in
    the reference; weight format "mxfp4_mx" of `fused_moe`): the experts are
    zero-padded along K at load to the MX kernel's multiple of 512.
    """

    is_monolithic = True
    supports_internal_mk = False

    def __init__(self, moe_config=None, mx_activations=None):
        self.moe = moe_config
        self.mx_activations = envs.QMOE_MXFP4_MX_ACTIVATIONS if mx_activations is None else bool(mx_activations)

    def maybe_roundup_sizes(self, hidden_size, intermediate_size_per_partition, *args, **kwargs):
        return hidden_size, intermediate_size_per_partition

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        if H % 32 or I % 32:
            raise ValueError(f"MXFP4 MoE sizes must be multiples of 32, got H={H}, I={I}")
        u8 = torch.uint8
        layer.register_parameter("w13_weight", _param(torch.empty(E, 2 * I, H // 2, dtype=u8)))
        layer.register_parameter("w13_weight_scale", _param(torch.empty(E, 2 * I, H // 32, dtype=u8)))
        layer.register_parameter("w2_weight", _param(torch.empty(E, H, I // 2, dtype=u8)))
        layer.register_parameter("w2_weight_scale", _param(torch.empty(E, H, I // 32, dtype=u8)))
        layer.register_parameter("w13_bias", _param(torch.zeros(E, 2 * I, dtype=torch.bfloat16)))
        layer.register_parameter("w2_bias", _param(torch.zeros(E, H, dtype=torch.bfloat16)))

    def process_weights_after_loading(self, layer):
        if getattr(layer, "_qmoe_processed", False):
            return
        moe_cfg = getattr(layer, "moe_config", None)
        if moe_cfg is not None and getattr(moe_cfg, "has_bias", True) is False:
            raise AssertionError("MXFP4 quantization requires bias.")
        dev = _device()
        act = _activation(layer)
        w13 = layer.w13_weight.data.to(dev).view(torch.uint8)
        s13 = layer.w13_weight_scale.data.to(dev).view(torch.uint8)
        b13 = layer.w13_bias.data.to(dev) if getattr(layer, "w13_bias", None) is not None else None
        if act == "swigluoai":  # [g0, u0, g1, u1, ...] -> [g | u]
            w13 = torch.cat([w13[:, 0::2], w13[:, 1::2]], dim=1)
            s13 = torch.cat([s13[:, 0::2], s13[:, 1::2]], dim=1)
            if b13 is not None:
                b13 = torch.cat([b13[:, 0::2], b13[:, 1::2]], dim=1)
        w2 = layer.w2_weight.data.to(dev).view(torch.uint8)
        s2 = layer.w2_weight_scale.data.to(dev).view(torch.uint8)
        if self.mx_activations:
            w13, s13 = _pad_experts_for_mx(w13, s13)
            w2, s2 = _pad_experts_for_mx(w2, s2)
        layer.w13_weight = _param(w13.contiguous())
        layer.w13_weight_scale = _param(s13.contiguous())
        layer.w2_weight = _param(w2.contiguous())
        layer.w2_weight_scale = _param(s2.contiguous())
        layer.w13_bias = _param(b13.to(torch.float32).contiguous()) if b13 is not None else None
        if getattr(layer, "w2_bias", None) is not None:
            layer.w2_bias = _param(layer.w2_bias.data.to(dev, torch.float32).contiguous())
        layer._qmoe_activation = act
        layer._qmoe_processed = True

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """`mxfp4.py:322-364`: route, then the fused MoE on MXFP4 experts."""
        return moe_forward(layer, x, router_logits, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale,
                           layer.w2_weight_scale, getattr(layer, "w13_bias", None), getattr(layer, "w2_bias", None),
                           "mxfp4_mx" if self.mx_activations else "mxfp4",
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS, input_ids=input_ids)


def _pad_experts_for_mx(w, s):
    """[E, N, K/2] codes + [E, N, K/32] e8m0 -> zero-padded along K to the MX
    kernel's multiple of 512 (one expert at a time)."""
    E, N, kb = w.shape
    wp, sp = pad_mxfp4_for_mx(w[0], s[0])
    out_w = torch.empty((E, N, wp.shape[1]), dtype=torch.uint8, device=w.device)
    out_s = torch.empty((E, N, sp.shape[1]), dtype=torch.uint8, device=w.device)
    out_w[0], out_s[0] = wp, sp
    for e in range(1, E):
        out_w[e], out_s[e] = pad_mxfp4_for_mx(w[e], s[e])
    return out_w, out_s
