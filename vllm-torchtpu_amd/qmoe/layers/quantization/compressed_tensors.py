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
                           group_size=d.get("group_size"), actorder=d.get("actorder"),
                           dynamic=d.get("dynamic", False), block_structure=d.get("block_structure"))


def _kind(v) -> str:
    """The lower-case name of an enum or string field ("float", "group", ...)."""
    return str(getattr(v, "value", v)).lower()


def _is_weight_fp8(q) -> bool:
    """`compressed_tensors.py:63-68`."""
    return q is not None and _kind(q.type) == "float" and int(q.num_bits) == 8


def _is_int4_w4aN(q) -> bool:
    """`compressed_tensors.py:71-83`: static INT4 weights, group or channel
    strategy."""
    return (q is not None and int(q.num_bits) == 4 and _kind(q.type) == "int"
            and _kind(q.strategy) in ("group", "channel") and not bool(getattr(q, "dynamic", False)))


def _is_mxfp4(q) -> bool:
    """MXFP4 weights (upstream compressed-tensors' MXFP4 scheme: 4-bit floats,
    group strategy, 32 values per e8m0 scale)."""
    return (q is not None and int(q.num_bits) == 4 and _kind(q.type) == "float"
            and _kind(q.strategy) == "group" and int(getattr(q, "group_size", 0) or 0) == 32)


def _build_fp8_config(weight_quant, input_quant):
    """`compressed_tensors.py:86-109`: an FP8 compressed-tensors scheme as an
    Fp8Config (block size from the block strategy, per-channel flag from the
    channel strategy; dynamic activations unless the scheme says static)."""
    from qmoe.layers.quantization.fp8 import Fp8Config

    block = weight_quant.block_structure if _kind(weight_quant.strategy) == "block" else None
    scheme = "dynamic" if (input_quant is None or bool(getattr(input_quant, "dynamic", True))) else "static"
    cfg = Fp8Config(is_checkpoint_fp8_serialized=True, activation_scheme=scheme, weight_block_size=block)
    cfg.is_channel_quant = _kind(weight_quant.strategy) == "channel"
    return cfg


class CompressedTensorsConfig:
    """The compressed-tensors schemes on this hot path
    (`compressed_tensors.py:200-254`, `compressed_tensors_moe.py:80-116`):
    FP8 linears through the FP8 linear method (the reference's bypass), and
    MoE experts dispatched by weight scheme -- packed INT4 (W4A16), MXFP4
    (W4A16, `compressed_tensors_moe_w4an_mxfp4.py`) or FP8 (the FP8 MoE
    method). The scheme of the checkpoint's first config group applies to
    every layer not in ``ignore``."""

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
        from qmoe.layers.quantization.fp8 import Fp8LinearMethod, Fp8MoEMethod
        from qmoe.layers.quantization.unquantized import UnquantizedFusedMoEMethod, UnquantizedLinearMethod

        moe = hasattr(layer, "moe_config")
        if any(prefix.startswith(p) for p in self.ignore) or self.weight_quant is None:
            return UnquantizedFusedMoEMethod(layer.moe_config) if moe else UnquantizedLinearMethod()
        wq, iq = self.weight_quant, self.input_quant
        if not moe:
            if _is_weight_fp8(wq):  # `compressed_tensors.py:227-231`
                return Fp8LinearMethod(_build_fp8_config(wq, iq))
            raise NotImplementedError("Compressed-tensors linear schemes other than FP8 are not implemented "
                                      "(the reference raises for them too)")
        if _is_int4_w4aN(wq):
            return CompressedTensorsW4A16MoEMethod(wq, iq, layer.moe_config)
        if _is_mxfp4(wq):
            return CompressedTensorsW4ANMxfp4MoEMethod(layer.moe_config)
        if _is_weight_fp8(wq):
            return Fp8MoEMethod(_build_fp8_config(wq, iq), layer.moe_config)
        raise RuntimeError(f"Unsupported TPU FusedMoe scheme: {wq}, {iq}")


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


class CompressedTensorsW4ANMxfp4MoEMethod:
    """Compressed-tensors MXFP4 MoE (`compressed_tensors_moe_w4an_mxfp4.py:
    49-342`), W4A16: bf16 activations against e2m1 experts expanded in
    registers with their e8m0 block scales.

    The checkpoint holds N-major e2m1 codes packed two per byte along K and
    one e8m0 byte per 32 K values (``w13_weight_packed u8 [E, 2I, H/2]``,
    ``w13_weight_scale u8 [E, 2I, H/32]``, ``w2_weight_packed u8 [E, H,
    I/2]``, ``w2_weight_scale u8 [E, H, I/32]``), no biases. The reference
    turns them into K-major native fp4 with float32 scales ``[E, K/32, 1,
    N]`` (`:173-273`); here they stay as loaded -- the same values: codes
    times 2^(byte - 127) -- and run as this package's ``mxfp4`` format. The
    scales of an unloaded intermediate padding are zeroed first, as the
    reference does (`:138-171`: an untouched 0xff byte would make a padded
    zero weight NaN). Requantizing to W4A8 (``MOE_REQUANTIZE_BLOCK_SIZE``)
    is not built and raises.

    ``mx_activations`` (default: the QMOE_MXFP4_MX_ACTIVATIONS flag) opts
    into MX-quantized activations (the W4A4 the method's name promises; no
    counterpart in the reference, which runs W4A16): experts zero-padded
    along K at load, weight format "mxfp4_mx" of `fused_moe`."""

    is_monolithic = True
    supports_internal_mk = False

    def __init__(self, moe_config=None, mx_activations=None):
        self.moe = moe_config
        self.group_size = 32
        self.mx_activations = envs.QMOE_MXFP4_MX_ACTIVATIONS if mx_activations is None else bool(mx_activations)

    def maybe_roundup_sizes(self, hidden_size, intermediate_size_per_partition, *args, **kwargs):
        return hidden_size, intermediate_size_per_partition

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        if H % 32 or I % 32:
            raise ValueError(f"MXFP4 MoE sizes must be multiples of 32, got H={H}, I={I}")
        u8 = torch.uint8
        layer.register_parameter("w13_weight_packed", _param(torch.empty(E, 2 * I, H // 2, dtype=u8)))
        layer.register_parameter("w13_weight_scale", _param(torch.empty(E, 2 * I, H // 32, dtype=u8)))
        layer.register_parameter("w2_weight_packed", _param(torch.empty(E, H, I // 2, dtype=u8)))
        layer.register_parameter("w2_weight_scale", _param(torch.empty(E, H, I // 32, dtype=u8)))

    def _neutralize_padded_scales(self, layer, s13, s2):
        """`compressed_tensors_moe_w4an_mxfp4.py:138-171`."""
        moe = getattr(layer, "moe_config", None) or self.moe
        unpadded = getattr(moe, "intermediate_size_per_partition_unpadded", None)
        padded = s2.shape[-1] * self.group_size
        if unpadded is None or unpadded >= padded:
            return
        if unpadded % self.group_size:
            raise ValueError("MXFP4 unpadded intermediate size per partition must be divisible by "
                             f"{self.group_size}, got {unpadded}.")
        s13[:, unpadded:padded, :] = 0
        s13[:, padded + unpadded:2 * padded, :] = 0
        s2[:, :, unpadded // self.group_size:] = 0

    def process_weights_after_loading(self, layer):
        if getattr(layer, "_qmoe_processed", False):
            return
        if envs.MOE_REQUANTIZE_BLOCK_SIZE:
            raise NotImplementedError("qmoe runs compressed-tensors MXFP4 experts as W4A16 at their 32-value "
                                      "blocks; W4A8 requantization (MOE_REQUANTIZE_BLOCK_SIZE) is not built")
        dev = _device()
        w13 = layer.w13_weight_packed.data.to(dev).view(torch.uint8).contiguous()
        w2 = layer.w2_weight_packed.data.to(dev).view(torch.uint8).contiguous()
        s13 = layer.w13_weight_scale.data.to(dev).view(torch.uint8).contiguous()
        s2 = layer.w2_weight_scale.data.to(dev).view(torch.uint8).contiguous()
        self._neutralize_padded_scales(layer, s13, s2)
        if self.mx_activations:
            from qmoe.layers.quantization.mxfp4 import _pad_experts_for_mx

            w13, s13 = _pad_experts_for_mx(w13, s13)
            w2, s2 = _pad_experts_for_mx(w2, s2)
        for name in ("w13_weight_packed", "w2_weight_packed"):
            delattr(layer, name)
        layer.w13_weight, layer.w2_weight = _param(w13), _param(w2)
        layer.w13_weight_scale, layer.w2_weight_scale = _param(s13), _param(s2)
        layer.w13_bias = None
        layer.w2_bias = None
        layer._qmoe_activation = _activation(layer)
        layer._qmoe_processed = True

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """`compressed_tensors_moe_w4an_mxfp4.py:275-342`: route, then the
        fused MoE with padded tokens skipped (the reference passes
        ``skip_padded_tokens=True``)."""
        return moe_forward(layer, x, router_logits, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale,
                           layer.w2_weight_scale, None, None, "mxfp4_mx" if self.mx_activations else "mxfp4",
                           skip_padded_tokens=True, input_ids=input_ids)

