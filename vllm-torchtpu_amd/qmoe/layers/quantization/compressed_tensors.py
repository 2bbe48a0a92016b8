"""Compressed-tensors packed-INT4 W4A16 MoE (the reference's
`layers/adapter/quantization/compressed_tensors/compressed_tensors_moe/
compressed_tensors_moe_w4a16.py`).

The checkpoint holds symmetric 4-bit integers packed eight per int32 along K
(nibble = value + 8, value 8j + i in bits 4i of carrier j) and one scale per
``group_size`` K values:
``w13_weight_packed int32 [E, 2I, H/8]``, ``w13_weight_scale [E, 2I, H/group]``,
``w2_weight_packed int32 [E, H, I/8]``, ``w2_weight_scale [E, H, I/group]``.
The reference XORs the carriers to two's complement, transposes them K-major
and runs gmm_v2 with ``rhs_quant_dtype=int4`` (`:258-300, 380-405`); groups
below 256 K are dequantized in bf16 there (`kernels/megablox/gmm_v2.py:
452-462`). Here the carriers stay resident as loaded (N-major, offset binary)
and the kernels expand each weight to bf16(value * scale) in registers,
bf16 activations, f32 accumulation. Runtime scales: bf16 ``[E, N, K/group]``.
"""

from types import SimpleNamespace

import torch

from qmoe import envs
from qmoe.layers.fused_moe import moe_forward
from qmoe.layers.quantization.fp8 import _activation, _device, _param

_GROUPS = (32, 64, 128)


def _args(d):
    """A compressed-tensors QuantizationArgs-like view of a dict / object."""
    if d is None or not isinstance(d, dict):
        return d
    return SimpleNamespace(num_bits=d.get("num_bits", 4), type=d.get("type", "int"),
                           symmetric=d.get("symmetric", True), strategy=d.get("strategy", "group"),
                           group_size=d.get("group_size"), actorder=d.get("actorder"))


class CompressedTensorsConfig:
    """The compressed-tensors schemes on this hot path: packed-INT4 W4A16 MoE
    experts (`compressed_tensors_moe.py:80-110` dispatch); the reference's
    other compressed-tensors schemes run through upstream vLLM layers."""

    def __init__(self, weight_quant=None, input_quant=None, ignore=None):
        self.weight_quant = _args(weight_quant)
        self.input_quant = _args(input_quant)
        self.ignore = ignore or []

    @classmethod
    def get_name(cls):
        return "compressed-tensors"

    @classmethod
    def from_config(cls, config: dict):
        groups = config.get("config_groups", {})
        first = next(iter(groups.values()), {})
        return cls(first.get("weights"), first.get("input_activations"), config.get("ignore"))

    def get_quant_method(self, layer, prefix=""):
        from qmoe.layers.quantization.unquantized import UnquantizedFusedMoEMethod, UnquantizedLinearMethod

        moe = hasattr(layer, "moe_config")
        if any(prefix.startswith(p) for p in self.ignore):
            return UnquantizedFusedMoEMethod(layer.moe_config) if moe else UnquantizedLinearMethod()
        if not moe:
            raise NotImplementedError("qmoe runs compressed-tensors MoE experts only; dense compressed-tensors "
                                      "schemes are not on this path")
        return CompressedTensorsW4A16MoEMethod(self.weight_quant, self.input_quant, layer.moe_config)


class CompressedTensorsW4A16MoEMethod:
    """Packed-INT4 W4A16 fused MoE (`compressed_tensors_moe_w4a16.py:60-405`)."""

    is_monolithic = True
    supports_internal_mk = False
    supports_eplb = False

    def __init__(self, weight_quant, input_quant=None, moe_config=None, layer_name=None):
        self.weight_quant = _args(weight_quant)
        self.input_quant = _args(input_quant)
        self.moe = moe_config
        self.num_bits = int(getattr(self.weight_quant, "num_bits", 4))
        self.packed_factor = 32 // self.num_bits
        self.strategy = getattr(self.weight_quant, "strategy", "group")
        gs = getattr(self.weight_quant, "group_size", None)
        self.group_size = -1 if gs is None else int(gs)

    def get_fused_moe_quant_config(self, layer):
        return None

    def _validate_w4a16_scheme(self):
        """`compressed_tensors_moe_w4a16.py:142-158`."""
        q = self.weight_quant
        num_bits = int(q.num_bits)
        qtype = getattr(q, "type", None)
        if qtype is None or "int" not in str(qtype).lower() or num_bits != 4:
            raise NotImplementedError("TPU W4A16 MoE supports integer INT4 weights only; "
                                      f"received quantization type {qtype!r}. num_bits {num_bits}")
        if not bool(getattr(q, "symmetric", False)):
            raise NotImplementedError("TPU W4A16 MoE currently supports symmetric INT4 only.")

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        """`compressed_tensors_moe_w4a16.py:172-260` (checkpoint shapes)."""
        self._validate_w4a16_scheme()
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        if self.strategy == "channel":
            raise NotImplementedError("qmoe runs INT4 experts with group scales (32, 64 or 128 K values); "
                                      "channel-strategy INT4 (one scale per row) is not supported")
        if self.group_size is None or self.group_size <= 0:
            raise ValueError(f"Invalid group_size for W4A16 MoE: {self.group_size}")
        if H % self.group_size != 0 or I % self.group_size != 0:
            raise ValueError(f"hidden_size ({H}) and intermediate_size_per_partition ({I}) must be divisible by "
                             f"group_size ({self.group_size})")
        if self.group_size not in _GROUPS:
            raise NotImplementedError(f"qmoe runs INT4 groups of {_GROUPS} K values, got {self.group_size}")
        g, pf, i32 = self.group_size, self.packed_factor, torch.int32
        layer.num_groups_w13, layer.num_groups_w2 = H // g, I // g
        layer.register_parameter("w13_weight_packed", _param(torch.empty(E, 2 * I, H // pf, dtype=i32)))
        layer.register_parameter("w2_weight_packed", _param(torch.empty(E, H, I // pf, dtype=i32)))
        layer.register_parameter("w13_weight_scale", _param(torch.empty(E, 2 * I, H // g, dtype=params_dtype)))
        layer.register_parameter("w2_weight_scale", _param(torch.empty(E, H, I // g, dtype=params_dtype)))
        layer.register_parameter("w13_weight_shape", _param(torch.empty(E, 2)))
        layer.register_parameter("w2_weight_shape", _param(torch.empty(E, 2)))

    def _validate_int32_weight_carriers(self, layer):
        """`compressed_tensors_moe_w4a16.py:160-170`."""
        for name in ("w13_weight_packed", "w2_weight_packed"):
            if not hasattr(layer, name):
                raise ValueError(f"Missing required W4A16 parameter: {name}.")
            if getattr(layer, name).dtype != torch.int32:
                raise NotImplementedError("TPU W4A16 MoE requires INT4 weights packed in INT32; "
                                          f"{name} has dtype {getattr(layer, name).dtype}.")

    def process_weights_after_loading(self, layer):
        """`compressed_tensors_moe_w4a16.py:302-355`, without the K-major
        transpose and sign flip (the kernels read the checkpoint form)."""
        if getattr(layer, "_qmoe_processed", False):
            return
        self._validate_w4a16_scheme()
        self._validate_int32_weight_carriers(layer)
        if envs.MOE_REQUANTIZE_BLOCK_SIZE or (envs.MOE_REQUANTIZE_WEIGHT_DTYPE or ""):
            raise NotImplementedError("qmoe runs INT4 experts at their checkpoint groups; unset "
                                      "MOE_REQUANTIZE_BLOCK_SIZE / MOE_REQUANTIZE_WEIGHT_DTYPE")
        dev = _device()
        for w, s in (("w13_weight_packed", "w13_weight_scale"), ("w2_weight_packed", "w2_weight_scale")):
            setattr(layer, w, _param(getattr(layer, w).data.to(dev).contiguous()))
            setattr(layer, s, _param(getattr(layer, s).data.to(dev, torch.bfloat16).contiguous()))
        layer.w13_bias = None
        layer.w2_bias = None
        layer._qmoe_activation = _activation(layer)
        layer._qmoe_processed = True

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """`compressed_tensors_moe_w4a16.py:357-405`: route, then the fused
        MoE on the packed-int4 experts."""
        return moe_forward(layer, x, router_logits, layer.w13_weight_packed, layer.w2_weight_packed,
                           layer.w13_weight_scale, layer.w2_weight_scale, None, None, "int4",
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS, input_ids=input_ids)
