"""FP8 / INT8 quant config and methods (the reference's
`layers/adapter/quantization/fp8.py`).

Same contract as the reference's `VllmFp8Config` (`:662-768`),
`VllmFp8LinearMethodTPU` (`:1342-1704`) and `VllmFp8MoEMethodTPU`
(`:771-1222`): vLLM-style ``create_weights`` registers the checkpoint
parameters, ``process_weights_after_loading`` converts them to the runtime
layout once, and ``apply`` / ``apply_monolithic`` run the forward.

Runtime layouts here (chosen for the MI355X kernels; the reference flips
weights to K-major instead):

* dense weight ``[n_out, n_in]`` (N-major, the checkpoint layout), with
  - per-channel f32 scale ``[n_out]`` (default: the checkpoint is dequantized
    to f32 and requantized per output channel, as the reference does,
    `:297-348`), or
  - with ``ENABLE_QUANTIZED_MATMUL_KERNEL=1 REQUANTIZE_BLOCK_SIZE=128``: a
    128x128-block checkpoint keeps its native codes and f32 tile scales
    ``[n_out/128, n_in/128]`` (no requantization); any other checkpoint is
    requantized per (output channel, 128-wide K block) -> ``[n_out, n_in/128]``.
  ``REQUANTIZE_WEIGHT_DTYPE=int8`` requantizes per channel to int8 (W8A8 with
  int8 activations, bit-exact int32 accumulation); ``float8_e5m2`` to e5m2
  codes (per channel: e5m2 activations as well, `util.py:80-124` quantizes
  them to the weight dtype; blocks of 512+: e4m3 activations, the grouped
  matmul's rule).
* MoE weights ``w13 [E, 2I, H]`` / ``w2 [E, H, I]``; a 128x128-block
  checkpoint keeps native codes + tile scales (the DeepSeek-V3 form), other
  checkpoints are requantized per channel.

Requantization runs the library's load-time quantizer kernel
(`qmoe_row_quant`, mode 1), which reproduces the reference's
`layers/core/quantization.py:232-318` bit for bit.
"""

import torch

from qmoe import envs, ops
from qmoe.layers.fused_moe import moe_forward
from qmoe.layers.linear_common import KEEP_VLLM_LAYOUT_ATTR, quantized_matmul

FP8 = torch.float8_e4m3fn
# requantization targets (`fp8.py:122-127`); the short names are the ones
# `ops.row_quant` takes
_REQUANT_DTYPES = {"float8_e4m3fn": FP8, "int8": torch.int8, "float8_e5m2": torch.float8_e5m2}
_QDTYPE_SHORT = {"float8_e4m3fn": "fp8", "int8": "int8", "float8_e5m2": "e5m2"}


# f32 bytes of one chunk of experts dequantized at load time
REQUANT_CHUNK_BYTES = 1 << 30


def _device():
    return torch.device("cuda", torch.cuda.current_device())


def _param(t):
    return torch.nn.Parameter(t, requires_grad=False)


def get_linear_quant_config():
    """(dtype name, torch dtype, block size or None, blockwise kernel) from
    the env gates, with the reference's validation (`fp8.py:216-267`)."""
    enable = envs.ENABLE_QUANTIZED_MATMUL_KERNEL
    block = envs.REQUANTIZE_BLOCK_SIZE
    name = envs.REQUANTIZE_WEIGHT_DTYPE
    if enable and not block:
        raise ValueError(
            "You should set REQUANTIZE_BLOCK_SIZE to enable quantized matmul kernel. "
            "Please set the value or disable the quantized matmul kernel."
        )
    if not enable and block:
        raise ValueError(
            "Blockwise quantization is supported by quantized matmul kernel. Please enable "
            "quantized_matmul_kernel or unset the quantize block size to trigger per-channel "
            "quantization."
        )
    if name not in _REQUANT_DTYPES:
        supported = ", ".join(sorted(_REQUANT_DTYPES))
        raise ValueError(f"Unsupported REQUANTIZE_WEIGHT_DTYPE={name!r}. Supported values: {supported}.")
    if block is not None:
        _check_block(block, "REQUANTIZE_BLOCK_SIZE")
        if block == 128 and name != "float8_e4m3fn":
            raise NotImplementedError("128-column blocks are dequantized to bf16 before the matmul; qmoe "
                                      "runs that regime for float8_e4m3fn codes only")
    return name, _REQUANT_DTYPES[name], block, bool(enable)


def _check_block(block, env_name):
    """Requantization blocks the kernels run: 128 (dequantized to bf16 before
    the matmul, the reference's regime for blocks under 256) or a
    power-of-two multiple of 512 (the quantized-activation regime)."""
    ok = block == 128 or (block >= 512 and block % 512 == 0 and ((block // 512) & (block // 512 - 1)) == 0)
    if not ok:
        raise NotImplementedError(f"qmoe runs {env_name}=128 or a power-of-two multiple of 512, got {block}")


def get_moe_quant_config():
    """(dtype name, torch dtype, block size or None) for FP8 MoE
    requantization from MOE_REQUANTIZE_WEIGHT_DTYPE / MOE_REQUANTIZE_BLOCK_SIZE,
    `fp8.py:185-213` (default: float8_e4m3fn per channel)."""
    name = envs.MOE_REQUANTIZE_WEIGHT_DTYPE or "float8_e4m3fn"
    block = envs.MOE_REQUANTIZE_BLOCK_SIZE or None
    if name not in _REQUANT_DTYPES:
        supported = ", ".join(sorted(_REQUANT_DTYPES))
        raise ValueError(f"Unsupported MOE_REQUANTIZE_WEIGHT_DTYPE={name!r}. Supported values: {supported}.")
    if block is not None:
        _check_block(block, "MOE_REQUANTIZE_BLOCK_SIZE")
        if block == 128 and name != "float8_e4m3fn":
            raise NotImplementedError("128-column blocks are dequantized to bf16 before the matmul; qmoe "
                                      "runs that regime for float8_e4m3fn codes only")
    return name, _REQUANT_DTYPES[name], block


def dequantize_fp8_weight(weight, weight_scale=None, weight_scale_inv=None, block=None,
                          logical_widths=None):
    """Checkpoint FP8 weight [N, K] -> f32, `fp8.py:132-182`: block scale
    (tile of ``block``), per-tensor / per-shard / per-channel scale."""
    w = weight.to(torch.float32)
    if block is not None:
        bh, bw = block
        n, k = w.shape
        s = weight_scale_inv.to(torch.float32)
        if n % bh == 0 and k % bw == 0:
            return (w.reshape(n // bh, bh, k // bw, bw) * s[:, None, :, None]).reshape(n, k)
        s = s.repeat_interleave(bh, 0).repeat_interleave(bw, 1)[:n, :k]
        return w * s
    s = weight_scale.to(torch.float32)
    if s.numel() > 1 and logical_widths is not None and s.numel() == len(logical_widths):
        s = s.repeat_interleave(torch.tensor(logical_widths, device=s.device)).unsqueeze(1)
    elif s.dim() == 1 and s.numel() == w.shape[0]:
        s = s.unsqueeze(1)
    return w * s


def requantize(w_f32, qdtype_name, block=None):
    """f32 [..., N, K] -> codes + scale with the load-time quantizer kernel
    (`layers/core/quantization.py:232-318`): per row ([.., N] scale) or per
    (row, B-column block) ([.., N, K/B]; B = 128 in one launch, larger B as
    rows of B columns)."""
    lead = w_f32.shape[:-1]
    k = w_f32.shape[-1]
    qd = _QDTYPE_SHORT[qdtype_name]
    if block is not None and k % block:
        raise ValueError(f"Quantization expects the requested axis to be divisible by block_size {block}, got {k}")
    if block is not None and block != 128:
        q, s = ops.row_quant(w_f32.reshape(-1, block).contiguous(), qd, mode="load")
        return q.reshape(*lead, k), s.reshape(*lead, k // block)
    q, s = ops.row_quant(w_f32.reshape(-1, k).contiguous(), qd, block=block, mode="load")
    q = q.reshape(*lead, k)
    s = s.reshape(*lead) if block is None else s.reshape(*lead, k // block)
    return q, s


class Fp8Config:
    """Quant config for FP8 checkpoints (`fp8.py:662-768`)."""

    def __init__(self, is_checkpoint_fp8_serialized=True, activation_scheme="dynamic",
                 weight_block_size=None, ignored_layers=None):
        if activation_scheme != "dynamic":
            raise ValueError(f"Unsupported activation scheme {activation_scheme}")
        self.is_checkpoint_fp8_serialized = is_checkpoint_fp8_serialized
        self.activation_scheme = activation_scheme
        self.weight_block_size = list(weight_block_size) if weight_block_size else None
        self.ignored_layers = ignored_layers or []
        # one scale per output channel in the checkpoint (compressed-tensors
        # channel strategy, `compressed_tensors.py:86-109`)
        self.is_channel_quant = False

    @classmethod
    def get_name(cls):
        return "fp8"

    @classmethod
    def from_config(cls, config: dict):
        method = config.get("quant_method", "")
        return cls(
            is_checkpoint_fp8_serialized="fp8" in method,
            activation_scheme=config.get("activation_scheme", "dynamic"),
            weight_block_size=config.get("weight_block_size"),
            ignored_layers=config.get("ignored_layers"),
        )

    def get_quant_method(self, layer, prefix=""):
        from qmoe.layers.quantization.unquantized import UnquantizedLinearMethod

        if any(prefix.startswith(p) for p in self.ignored_layers):
            return UnquantizedLinearMethod()
        if hasattr(layer, "moe_config"):
            return Fp8MoEMethod(self, layer.moe_config)
        return Fp8LinearMethod(self)


class Fp8LinearMethod:
    """Dense FP8 / INT8 linear (`fp8.py:1342-1704`)."""

    def __init__(self, quant_config: Fp8Config):
        self.quant_config = quant_config
        self.weight_block_size = quant_config.weight_block_size
        self.block_quant = self.weight_block_size is not None
        self.w8a16_max_rows = envs.TPU_FP8_LINEAR_W8A16_MAX_ROWS
        self._linear_quant_config = get_linear_quant_config()

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size,
                       output_size, params_dtype, **extra_weight_attrs):
        n = sum(output_partition_sizes)
        k = input_size_per_partition
        layer.logical_widths = list(output_partition_sizes)
        layer.input_size_per_partition = k
        layer.output_size_per_partition = n
        layer.orig_dtype = params_dtype
        wdt = FP8 if self.quant_config.is_checkpoint_fp8_serialized else params_dtype
        layer.register_parameter("weight", _param(torch.empty(n, k, dtype=wdt)))
        if self.quant_config.is_checkpoint_fp8_serialized:
            if self.block_quant:
                bh, bw = self.weight_block_size
                s = torch.empty((n + bh - 1) // bh, (k + bw - 1) // bw, dtype=torch.float32)
                layer.register_parameter("weight_scale_inv", _param(s))
            elif getattr(self.quant_config, "is_channel_quant", False):
                layer.register_parameter("weight_scale", _param(torch.empty(n, 1, dtype=torch.float32)))
            else:
                layer.register_parameter("weight_scale", _param(torch.empty(len(output_partition_sizes),
                                                                            dtype=torch.float32)))
        for name, v in extra_weight_attrs.items():
            setattr(layer.weight, name, v)

    def process_weights_after_loading(self, layer):
        """Checkpoint -> runtime FP8/INT8 (`fp8.py:1535-1667`), once."""
        if getattr(layer, "_qmoe_processed", False):
            return
        name, _, block, blockwise = self._linear_quant_config
        if _is_embedding(layer):
            # embedding tables are gathered by row: one scale per row
            block, blockwise = None, False
        dev = _device()
        weight = layer.weight.data.to(dev)
        ckpt_block = None
        if self.quant_config.is_checkpoint_fp8_serialized and self.block_quant:
            ckpt_block = tuple(getattr(layer, "weight_block_size", None) or self.weight_block_size)
        if (blockwise and block == 128 and envs.QMOE_FP8_NATIVE_BLOCKS and name == "float8_e4m3fn"
                and ckpt_block == (128, 128) and weight.dtype == FP8 and weight.shape[0] % 128 == 0
                and weight.shape[1] % 128 == 0):
            # opt-in: native 128x128 tiles, codes and tile scales as loaded
            # (the blockwise W8A8 recipe, compact [N/128, K/128] scales)
            w_rt = weight.contiguous()
            s_rt = layer.weight_scale_inv.data.to(dev, torch.float32).contiguous()
        else:
            if weight.dtype == FP8:
                w_f = dequantize_fp8_weight(
                    weight,
                    weight_scale=getattr(layer, "weight_scale", None),
                    weight_scale_inv=getattr(layer, "weight_scale_inv", None),
                    block=ckpt_block,
                    logical_widths=getattr(layer, "logical_widths", None),
                ) if ckpt_block or hasattr(layer, "weight_scale") else weight.to(torch.float32)
            else:
                w_f = weight.to(torch.float32)
            if block is not None and w_f.shape[-1] < block:
                block = None  # `fp8.py:332-337`: too narrow for the block
            w_rt, s_rt = requantize(w_f, name, block if blockwise else None)
            if blockwise and block is not None:
                # the reference's runtime layout [1, K/B, 1, N]
                # (`fp8.py:270-294`), as a view of the N-major [N, K/B] buffer
                s_rt = s_rt.t()[None, :, None, :]
        for attr in ("weight_scale_inv", "weight_scale"):
            if hasattr(layer, attr):
                delattr(layer, attr)
        layer.weight = _param(w_rt)
        layer.weight_scale = _param(s_rt)
        layer._qmoe_processed = True

    def apply(self, layer, x, bias=None):
        """`fp8.py:1669-1690`: quantized matmul, then the bias. The weight is
        held in vLLM's ``[n_out, n_in]`` layout for every layer, so a layer
        marked KEEP_VLLM_LAYOUT (read raw elsewhere) needs no flip here; the
        matmul takes the ``[n_in, n_out]`` view. An embedding table used as
        the output projection (VocabParallelEmbedding: tied lm_head) keeps
        bf16 activations (W8A16, `:1679-1681`)."""
        if _is_embedding(layer):
            x2 = x.reshape(-1, x.shape[-1])
            rows = max(1, x2.shape[0])
            out = quantized_matmul(x2, layer.weight.t(), layer.weight_scale, w8a16_max_rows=rows)
            out = out.reshape(*x.shape[:-1], out.shape[-1])
        else:
            out = quantized_matmul(x, layer.weight.t(), layer.weight_scale,
                                   w8a16_max_rows=self.w8a16_max_rows)
        if bias is not None:
            out = out + bias
        return out

    def embedding(self, layer, input_):
        """`fp8.py:1692-1698`: gather the rows of the ``[vocab, H]`` codes and
        their per-row scales, dequantize in the layer's dtype."""
        flat = input_.reshape(-1)
        out_dtype = getattr(layer, "params_dtype", None) or getattr(layer, "orig_dtype", None) or torch.bfloat16
        w = torch.index_select(layer.weight, 0, flat).to(out_dtype)
        s = torch.index_select(layer.weight_scale.reshape(-1), 0, flat).to(out_dtype).unsqueeze(-1)
        return (w * s).reshape(*input_.shape, -1)

    def tie_weights(self, layer, embed_tokens):
        """`fp8.py:1700-1704`: share the embedding's codes and scales."""
        layer.weight = embed_tokens.weight
        layer.weight_scale = embed_tokens.weight_scale
        setattr(layer, KEEP_VLLM_LAYOUT_ATTR, True)
        return layer


class Fp8MoEMethod:
    """FP8 fused MoE (`fp8.py:771-1222`), whole expert set on one GPU."""

    is_monolithic = True
    supports_internal_mk = False

    def __init__(self, quant_config: Fp8Config, moe_config=None):
        self.quant_config = quant_config
        self.moe = moe_config
        self.weight_block_size = quant_config.weight_block_size
        self.block_quant = self.weight_block_size is not None

    def maybe_roundup_sizes(self, hidden_size, intermediate_size_per_partition, *args, **kwargs):
        """No padding: the kernels take any H, I that are multiples of 128
        (block scales) or 32 (per-channel)."""
        return hidden_size, intermediate_size_per_partition

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **extra_weight_attrs):
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        wdt = FP8 if self.quant_config.is_checkpoint_fp8_serialized else params_dtype
        layer.register_parameter("w13_weight", _param(torch.empty(E, 2 * I, H, dtype=wdt)))
        layer.register_parameter("w2_weight", _param(torch.empty(E, H, I, dtype=wdt)))
        if self.quant_config.is_checkpoint_fp8_serialized:
            if self.block_quant:
                bh, bw = self.weight_block_size
                layer.register_parameter("w13_weight_scale_inv", _param(torch.empty(
                    E, (2 * I + bh - 1) // bh, (H + bw - 1) // bw, dtype=torch.float32)))
                layer.register_parameter("w2_weight_scale_inv", _param(torch.empty(
                    E, (H + bh - 1) // bh, (I + bw - 1) // bw, dtype=torch.float32)))
            elif getattr(self.quant_config, "is_channel_quant", False):
                layer.register_parameter("w13_weight_scale", _param(torch.ones(E, 2 * I, 1, dtype=torch.float32)))
                layer.register_parameter("w2_weight_scale", _param(torch.ones(E, H, 1, dtype=torch.float32)))
            else:
                layer.register_parameter("w13_weight_scale", _param(torch.ones(E, 2, dtype=torch.float32)))
                layer.register_parameter("w2_weight_scale", _param(torch.ones(E, dtype=torch.float32)))

    def process_weights_after_loading(self, layer):
        """Checkpoint -> runtime (`fp8.py:982-1106`), once. The FP8 MoE
        asserts no bias, as the reference does (`:994`).

        The reference's recipe (`fp8.py:486-617`): dequantize to f32 in
        chunks of experts, de-interleave swigluoai gate/up rows, zero the
        padding of an unpadded intermediate size and pad the intermediate
        size to a multiple of 128 (`:351-406`), requantize to
        MOE_REQUANTIZE_WEIGHT_DTYPE (float8_e4m3fn by default, int8 or float8_e5m2) per
        channel, or per (row, MOE_REQUANTIZE_BLOCK_SIZE columns). At run time
        per-channel and 512+ blocks take the quantized-activation recipe, 128
        blocks the bf16-dequantized one. With QMOE_FP8_NATIVE_BLOCKS=1 a
        128x128-block checkpoint keeps its tiles instead (the blockwise W8A8
        recipe of BASELINE config 4)."""
        if getattr(layer, "_qmoe_processed", False):
            return
        if getattr(layer, "w13_bias", None) is not None or getattr(layer, "w2_bias", None) is not None:
            raise AssertionError("FP8 MoE does not support bias")
        name, _, block = get_moe_quant_config()
        dev = _device()
        act = _activation(layer)
        interleaved = act == "swigluoai"
        w13 = layer.w13_weight.data.to(dev)
        w2 = layer.w2_weight.data.to(dev)
        E, N13, H = w13.shape
        I = w2.shape[2]
        if self.block_quant:
            bh, bw = self.weight_block_size
            for wname, t in (("w13_weight", w13), ("w2_weight", w2)):
                if t.shape[1] % bh or t.shape[2] % bw:
                    raise ValueError(
                        "FP8 block quantized MoE weights must be divisible by the checkpoint block size, "
                        f"got {wname}.shape={tuple(t.shape)} and block_size={tuple(self.weight_block_size)}.")
        native = (envs.QMOE_FP8_NATIVE_BLOCKS and block is None and name == "float8_e4m3fn" and self.block_quant
                  and tuple(self.weight_block_size) == (128, 128) and w13.dtype == FP8 and not interleaved
                  and N13 % 128 == 0 and H % 128 == 0 and I % 128 == 0)
        if native:
            layer.w13_weight = _param(w13.contiguous())
            layer.w2_weight = _param(w2.contiguous())
            layer.w13_weight_scale = _param(layer.w13_weight_scale_inv.data.to(dev, torch.float32).contiguous())
            layer.w2_weight_scale = _param(layer.w2_weight_scale_inv.data.to(dev, torch.float32).contiguous())
            layer._qmoe_format = "fp8_block"
        else:
            # the logical intermediate size (the rest of I is checkpoint
            # padding, zeroed) and its 128-aligned runtime size
            moe = getattr(layer, "moe_config", None) or self.moe
            real = getattr(moe, "intermediate_size_per_partition_unpadded", None) or I
            Ip = (I + 127) // 128 * 128
            for wname, kk in (("w13", H), ("w2", Ip)):
                if block is not None and kk % block:
                    raise ValueError(f"Unsupported MoE quantization: {wname} contracting dimension {kk} is not "
                                     f"divisible by block_size={block}.")
            qdt = _REQUANT_DTYPES[name]

            def alloc(n, k):
                return (torch.empty((E, n, k), dtype=qdt, device=dev),
                        torch.empty((E, n) if block is None else (E, n, k // block), dtype=torch.float32,
                                    device=dev))

            q13, s13 = alloc(2 * Ip, H)
            q2, s2 = alloc(H, Ip)
            # dequantize -> (de-interleave) -> zero / pad -> requantize on the
            # device, a chunk of experts at a time so the f32 copy stays under
            # ~1 GiB (the reference's chunked loop, `fp8.py:414-453`)
            chunk = max(1, REQUANT_CHUNK_BYTES // (4 * 2 * Ip * H))
            for e0 in range(0, E, chunk):
                e1 = min(E, e0 + chunk)
                f = self._dequant_experts(layer, "w13", w13[e0:e1], e0)
                if interleaved:  # `fp8.py:364-367`: [g0, u0, g1, u1, ...] -> [g | u]
                    f = torch.cat([f[:, 0::2], f[:, 1::2]], dim=1)
                g, u = f[:, :I], f[:, I:]
                f = torch.zeros((e1 - e0, 2 * Ip, H), dtype=torch.float32, device=dev)
                f[:, :real], f[:, Ip:Ip + real] = g[:, :real], u[:, :real]
                del g, u
                q13[e0:e1], s13[e0:e1] = requantize(f, name, block)
                f2 = torch.zeros((e1 - e0, H, Ip), dtype=torch.float32, device=dev)
                f2[:, :, :real] = self._dequant_experts(layer, "w2", w2[e0:e1], e0)[:, :, :real]
                q2[e0:e1], s2[e0:e1] = requantize(f2, name, block)
                del f, f2
            layer.w13_weight, layer.w2_weight = _param(q13), _param(q2)
            layer.w13_weight_scale, layer.w2_weight_scale = _param(s13), _param(s2)
            if block == 128:
                layer._qmoe_format = "fp8_w8a16"
            else:
                layer._qmoe_format = {"float8_e4m3fn": "fp8", "int8": "int8", "float8_e5m2": "e5m2"}[name]
        for attr in ("w13_weight_scale_inv", "w2_weight_scale_inv"):
            if hasattr(layer, attr):
                delattr(layer, attr)
        layer._qmoe_activation = act
        layer._qmoe_processed = True

    def _dequant_experts(self, layer, which, w, e0=0):
        """f32 copy of experts [e0, e0 + len(w)) of `which` (w13 / w2)."""
        if w.dtype != FP8:
            return w.to(torch.float32)
        n = w.shape[0]
        if self.block_quant:
            s = getattr(layer, f"{which}_weight_scale_inv").data[e0:e0 + n].to(w.device)
            return torch.stack([dequantize_fp8_weight(w[e], weight_scale_inv=s[e],
                                                      block=tuple(self.weight_block_size))
                                for e in range(n)])
        s = getattr(layer, f"{which}_weight_scale").data.to(w.device, torch.float32)
        if s.numel() > 1:
            s = s[e0:e0 + n]
        if which == "w13" and s.dim() == 2 and s.shape[1] == 2:  # one scale per w1 / w3 shard
            half = w.shape[1] // 2
            s = s.repeat_interleave(half, dim=1)[:, :, None]
        else:
            s = s.reshape(w.shape[0], -1, 1) if s.numel() > w.shape[0] else s.reshape(-1, 1, 1)
        return w.to(torch.float32) * s

    def apply_monolithic(self, layer, x, router_logits, input_ids=None):
        """`fp8.py:1108-1222` (single-GPU branch): route, then fused MoE; an
        armed layer (`arm_fused_moe_decode`) returns shared + routed from the
        fused decode op (`fp8.py:1203-1220`)."""
        from qmoe.layers import fused_moe_decode as fmd

        if fmd.fused_moe_decode_supported(self):
            from qmoe.layers import moe_routing

            # zero-weight (padding) routes add nothing to the op's sums, so
            # TPU_MOE_SKIP_PADDED_TOKENS needs no mask here
            out = fmd.fused_moe_decode_routed(self, layer, x, router_logits, input_ids=input_ids)
            if out is not None:
                return out
            topk_weights, topk_ids = moe_routing.route(layer, x, router_logits, input_ids=input_ids)
            return fmd.fused_moe_decode(self, layer, x, topk_weights, topk_ids)
        return moe_forward(layer, x, router_logits, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale,
                           layer.w2_weight_scale, None, None, layer._qmoe_format,
                           skip_padded_tokens=envs.TPU_MOE_SKIP_PADDED_TOKENS, input_ids=input_ids)


def _is_embedding(layer) -> bool:
    """A vocab embedding table (vLLM's VocabParallelEmbedding or a subclass,
    e.g. ParallelLMHead), `fp8.py:1612-1614, 1679`."""
    return any(c.__name__ == "VocabParallelEmbedding" for c in type(layer).__mro__) or bool(
        getattr(layer, "_qmoe_embedding", False))


def _activation(layer):
    act = getattr(layer, "activation", "silu")
    act = getattr(act, "value", act)  # vLLM passes an enum in newer versions
    return str(act).lower()
