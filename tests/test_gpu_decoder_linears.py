"""The other linears of the decoder layers the MoE configs come from, through
the same method boundary (`layers/adapter/quantization/fp8.py:1669-1690`
apply; the shared expert runs beside the routed layer, `:1170-1172`), at
their real shapes:

* DeepSeek-V3 attention projections from 128x128 FP8 checkpoints: q_a
  (7168 -> 1536), kv_a with the rope part (7168 -> 576, not a multiple of
  128: the checkpoint's last scale tile is partial), q_b (1536 -> 24576),
  kv_b (512 -> 32768), o (16384 -> 7168), and the shared expert's gate_up
  (7168 -> 4096) and down (2048 -> 7168) -- the reference's default recipe
  (dequantize, requantize per channel, per-token FP8 activations) and, where
  the tiles fit, this build's native-tile recipe;
* Llama-3-8B qkv (4096 -> 6144 as three shards with one tensor scale each,
  `logical_widths`) and o (4096 -> 4096);
* DeepSeek-V3's router gate (7168 -> 256), a bf16 linear
  (`UnquantizedLinearMethod`, `unquantized.py:88-146`).

Weight codes and scales are checked bit-exactly against the oracle's
load-time transforms; outputs of sampled rows against the oracle's forward
with the north-star row bar."""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows, assert_close_same_codes
from oracle import codecs, linear, quant

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _tile_checkpoint(rng, N, K):
    """A 128x128-tile FP8 checkpoint of randn * 0.02 weights: codes [N, K]
    and weight_scale_inv [ceil(N/128), ceil(K/128)] (rows past N are
    quantized with the last tile and dropped, as a checkpoint of an
    unaligned projection holds them)."""
    Np, Kp = -(-N // 128) * 128, -(-K // 128) * 128
    w = np.zeros((Np, Kp), np.float32)
    w[:N, :K] = rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.02)
    codes, s_inv = quant.quantize_fp8_tiles(w)
    return np.ascontiguousarray(codes[:N, :K]), s_inv


def _dequant_ckpt(codes, s_inv):
    """`fp8.py:132-182` (block branch, float32 out): each code times the
    scale of its tile, the scale grid repeated and cut to [N, K]."""
    n, k = codes.shape
    s = np.repeat(np.repeat(s_inv, 128, axis=0), 128, axis=1)[:n, :k]
    return (codecs.e4m3_decode(codes) * s).astype(np.float32)


def _rows(M, n=6):
    return np.unique(np.linspace(0, M - 1, min(M, n)).round().astype(np.int64))


def _env(monkeypatch, native):
    for v in ("ENABLE_QUANTIZED_MATMUL_KERNEL", "REQUANTIZE_BLOCK_SIZE", "REQUANTIZE_WEIGHT_DTYPE",
              "QMOE_FP8_NATIVE_BLOCKS"):
        monkeypatch.delenv(v, raising=False)
    if native:
        monkeypatch.setenv("ENABLE_QUANTIZED_MATMUL_KERNEL", "1")
        monkeypatch.setenv("REQUANTIZE_BLOCK_SIZE", "128")
        monkeypatch.setenv("QMOE_FP8_NATIVE_BLOCKS", "1")


# DeepSeek-V3: (name, N out, K in)
DSV3 = [("q_a", 1536, 7168), ("kv_a", 576, 7168), ("q_b", 24576, 1536), ("kv_b", 32768, 512),
        ("o", 7168, 16384), ("shared_gate_up", 4096, 7168), ("shared_down", 7168, 2048)]


@pytest.mark.parametrize("M", [1, 64, 512, 4096])
@pytest.mark.parametrize("name,N,K", DSV3)
def test_dsv3_projection_default_recipe(dev, monkeypatch, name, N, K, M):
    """Default recipe: checkpoint tiles dequantized in float32, requantized
    per output channel (`fp8.py:297-348`); apply = per-token FP8 activations
    x per-channel weights (`kernels/quantized_matmul/util.py:80-124`)."""
    from qmoe.layers import quantization as q

    print(f"dsv3 {name} N={N} K={K} M={M} default", flush=True)
    _env(monkeypatch, native=False)
    rng = np.random.default_rng(N + K)
    codes, s_inv = _tile_checkpoint(rng, N, K)
    method = q.Fp8LinearMethod(q.Fp8Config(weight_block_size=[128, 128]))
    layer = torch.nn.Module()
    method.create_weights(layer, K, [N], K, N, torch.bfloat16)
    assert tuple(layer.weight_scale_inv.shape) == s_inv.shape
    layer.weight.data = _t(codes, dev).view(torch.float8_e4m3fn)
    layer.weight_scale_inv.data = _t(s_inv, dev)
    method.process_weights_after_loading(layer)
    wq, ws = quant.quantize_tensor(_dequant_ckpt(codes, s_inv), "fp8")
    np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), wq)
    np.testing.assert_array_equal(layer.weight_scale.cpu().numpy(), ws)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    y = method.apply(layer, _t(x, dev, torch.bfloat16))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    r = _rows(M)
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, "fp8")
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"dsv3 {name} M={M}")


@pytest.mark.parametrize("M", [1, 256])
@pytest.mark.parametrize("name,N,K", [p for p in DSV3 if p[1] % 128 == 0 and p[2] % 128 == 0])
def test_dsv3_projection_native_tiles(dev, monkeypatch, name, N, K, M):
    """This build's opt-in native recipe (QMOE_FP8_NATIVE_BLOCKS=1 with the
    block-128 env): checkpoint codes and tile scales kept as loaded,
    per-(token, 128) FP8 activations, the reference's blockwise test oracle
    (`tests/kernels/test_quantized_matmul_kernel.py:66-94`)."""
    from qmoe.layers import quantization as q

    print(f"dsv3 {name} N={N} K={K} M={M} native tiles", flush=True)
    _env(monkeypatch, native=True)
    rng = np.random.default_rng(N + K + 1)
    codes, s_inv = _tile_checkpoint(rng, N, K)
    method = q.Fp8LinearMethod(q.Fp8Config(weight_block_size=[128, 128]))
    layer = torch.nn.Module()
    method.create_weights(layer, K, [N], K, N, torch.bfloat16)
    layer.weight.data = _t(codes, dev).view(torch.float8_e4m3fn)
    layer.weight_scale_inv.data = _t(s_inv, dev)
    method.process_weights_after_loading(layer)
    np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), codes)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    y = method.apply(layer, _t(x, dev, torch.bfloat16))
    r = _rows(M)
    ref, _, _ = linear.w8a8_blockwise(x[r], codes, linear.tile_scales_to_blocks(s_inv, N))
    assert_close_rows(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"dsv3 {name} native M={M}")


@pytest.mark.parametrize("M", [1, 16, 512, 4096])
@pytest.mark.parametrize("name,widths,K", [("qkv", [4096, 1024, 1024], 4096), ("o", [4096], 4096)])
def test_llama_attention_per_tensor_shards(dev, monkeypatch, name, widths, K, M):
    """Llama-3-8B FP8 checkpoints with one tensor scale per merged shard
    (`logical_widths`, `fp8.py:132-182` tensor branch) -> per-channel
    requant -> W8A8."""
    from qmoe.layers import quantization as q

    print(f"llama {name} widths={widths} K={K} M={M}", flush=True)
    _env(monkeypatch, native=False)
    rng = np.random.default_rng(K + len(widths) + M)
    N = sum(widths)
    w = rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.02)
    shard_scales = []
    codes = np.empty((N, K), np.uint8)
    o = 0
    for n in widths:  # per-tensor checkpoint scale of each shard
        s = np.float32(np.abs(w[o:o + n]).max() / 448.0)
        codes[o:o + n] = codecs.e4m3_encode(np.clip(w[o:o + n] / s, -448, 448).astype(np.float32))
        shard_scales.append(s)
        o += n
    shard_scales = np.array(shard_scales, np.float32)
    method = q.Fp8LinearMethod(q.Fp8Config())
    layer = torch.nn.Module()
    method.create_weights(layer, K, widths, K, N, torch.bfloat16)
    assert tuple(layer.weight_scale.shape) == (len(widths),)
    layer.weight.data = _t(codes, dev).view(torch.float8_e4m3fn)
    layer.weight_scale.data = _t(shard_scales, dev)
    method.process_weights_after_loading(layer)
    w_deq = codecs.e4m3_decode(codes) * np.repeat(shard_scales, widths)[:, None]
    wq, ws = quant.quantize_tensor(w_deq.astype(np.float32), "fp8")
    np.testing.assert_array_equal(layer.weight.view(torch.uint8).cpu().numpy(), wq)
    np.testing.assert_array_equal(layer.weight_scale.cpu().numpy(), ws)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    y = method.apply(layer, _t(x, dev, torch.bfloat16))
    r = _rows(M)
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, "fp8")
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"llama {name} M={M}")


@pytest.mark.parametrize("M", [1, 8, 64, 4096])
def test_dsv3_router_gate_bf16(dev, M):
    """The router gate (7168 -> 256 experts) stays bf16
    (`UnquantizedLinearMethod`): bf16 x bf16 with f32 accumulation."""
    from qmoe.layers.quantization.unquantized import UnquantizedLinearMethod

    print(f"dsv3 router gate M={M}", flush=True)
    rng = np.random.default_rng(M)
    N, K = 256, 7168
    w = codecs.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    method = UnquantizedLinearMethod()
    layer = torch.nn.Module()
    method.create_weights(layer, K, [N], K, N, torch.bfloat16)
    layer.weight.data = _t(w, dev, torch.bfloat16)
    method.process_weights_after_loading(layer)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    y = method.apply(layer, _t(x, dev, torch.bfloat16))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    r = _rows(M)
    ref = linear.w16a16(x[r], w)
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"router gate M={M}")
