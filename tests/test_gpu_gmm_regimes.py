"""GPU parity of the grouped matmul's two numeric regimes
(`kernels/megablox/gmm_v2.py:452-462, 500-548`):

* quantized-lhs (weights with quant blocks of 256+ columns, per-channel
  included): activations quantized per (row, 512 columns) in bf16
  arithmetic -- codes and scales bit-exact -- then the W8A8_GMM GEMM
  (streaming, FP8 tiled and generic tiled kernels, split-K, fused
  activation, grouped);
* dequantize-before-matmul (quant blocks under 256): W8A16_BLK, each weight
  bf16(code * bf16(scale)).
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows, assert_close_same_codes
from oracle import codecs, linear, quant
from oracle import moe as omoe

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _bf16(rng, shape, scale=1.0):
    return codecs.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("M,K", [(1, 4096), (7, 1152), (64, 7168), (300, 2048), (3, 640), (2, 14336)])
def test_gmm_quant_bit_exact(dev, qdtype, M, K):
    from qmoe import ops

    print(f"gmm quant {qdtype} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K)
    x = _bf16(rng, (M, K), 3.0)
    x[0, :] = 0.0  # zero row: every block keeps scale 0
    if M > 2:
        x[2, 5] = 1e4  # outlier in block 0 only
        x[1, min(K - 1, 600):] = 0.0  # a zero tail
    q_ref, s_ref = quant.quantize_gmm_lhs(x, qdtype)
    q, s = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype, mode="gmm")
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))


def _gmm_case(rng, M, K, N, qdtype):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    x = _bf16(rng, (M, K))
    x[:, : min(K, 512)] *= 30.0  # blocks with different scales
    return x, wq, ws


# (M, K, N): streaming (<= 32 rows), split-K streaming (tall K), the FP8 tiled
# kernel with 32/64/128-token tiles and a K split, ragged shapes
GMM_SHAPES = [(1, 4096, 1024), (5, 14336, 512), (32, 2048, 768), (33, 1024, 640), (96, 8192, 512),
              (200, 2048, 2304), (513, 1024, 1024), (130, 7168, 384)]


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("M,K,N", GMM_SHAPES)
def test_gmm_gemm_dense(dev, qdtype, M, K, N):
    from qmoe import _capi, ops

    print(f"gmm gemm {qdtype} M={M} K={K} N={N} plan "
          f"{ops.plan_for_shape(_capi.W8A8_GMM, M, N, K, wfmt=int(qdtype == 'int8'))}", flush=True)
    rng = np.random.default_rng(M * 3 + K + N)
    x, wq, ws = _gmm_case(rng, M, K, N, qdtype)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref, xq_ref, xs_ref = linear.w8a8_gmm(x, wq, ws, qdtype, bias=bias)
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype, mode="gmm")
    np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), xq_ref.view(np.uint8))
    y = ops.gemm(_capi.W8A8_GMM, xq.view(torch.uint8), _t(wq.view(np.uint8), dev), a_scale=xs,
                 w_scale=_t(ws, dev), wfmt=int(qdtype == "int8"), bias=_t(bias, dev))
    got = y.float().cpu().numpy()
    assert_close_same_codes(got, ref, f"gmm {qdtype} {M}x{K}x{N}")
    # the reference's own form accumulates the K/512 block results in bf16
    # (each addition rounds the accumulator): within that accumulation's
    # error, K/512 * 2^-8 of the row max, and the cosine bar
    nb = -(-K // 512)
    assert_close_rows(got, linear.w8a8_gmm_bf16acc(x, wq, ws, qdtype, bias=bias), "vs bf16 acc",
                      rel=max(2e-2, nb * 2.0 ** -8))


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("M,K,I", [(8, 2048, 256), (100, 8192, 320), (300, 1024, 384)])
def test_gmm_gemm_fused_activation(dev, qdtype, M, K, I):
    """gate/up with silu fused (the split-K finishing kernel applies the
    per-channel weight scale for the tiled FP8 kernel's K split)."""
    from qmoe import _capi, ops

    print(f"gmm act {qdtype} M={M} K={K} I={I}", flush=True)
    rng = np.random.default_rng(M + K + I)
    x, wq, ws = _gmm_case(rng, M, K, 2 * I, qdtype)
    gu, _, _ = linear.w8a8_gmm(x, wq, ws, qdtype, round_out=False)
    ref = codecs.bf16_round(omoe.act_fn(gu[:, :I], gu[:, I:], "silu"))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype, mode="gmm")
    y = ops.gemm(_capi.W8A8_GMM, xq.view(torch.uint8), _t(wq.view(np.uint8), dev), a_scale=xs,
                 w_scale=_t(ws, dev), wfmt=int(qdtype == "int8"), activation="silu")
    assert_close_rows(y.float().cpu().numpy(), ref, f"gmm act {qdtype}")


@pytest.mark.parametrize("M,K,N,bn", [(1, 2048, 512, 1), (16, 4096, 1024, 128), (64, 1024, 640, 1),
                                      (65, 2048, 768, 128), (300, 1024, 1024, 1), (200, 7168, 256, 128)])
def test_w8a16_block_dense(dev, M, K, N, bn):
    from qmoe import _capi, ops

    print(f"w8a16 blk M={M} K={K} N={N} bn={bn}", flush=True)
    rng = np.random.default_rng(M + K + N + bn)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if bn == 128:
        wq, st = quant.quantize_fp8_tiles(w)
        sblk = linear.tile_scales_to_blocks(st, N)
        s_dev = st
    else:
        wq, sblk = quant.quantize_tensor(w, "fp8", block=128)
        s_dev = sblk
    x = _bf16(rng, (M, K))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref = linear.w8a16_blockwise(x, wq, sblk, bias=bias)
    y = ops.gemm(_capi.W8A16_BLK, _t(x, dev, torch.bfloat16), _t(wq, dev), w_scale=_t(s_dev, dev), ws_bn=bn,
                 bias=_t(bias, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"w8a16 blk {M}x{K}x{N}")


def test_w8a16_block_one_hot_dequant_bit_exact(dev):
    """One-hot activation rows read single weights back: bf16(code *
    bf16(scale)) exactly (streaming M = 16, generic tiled M = 256), with
    scales whose mantissas make the products round."""
    from qmoe import _capi, ops

    rng = np.random.default_rng(8)
    K, N = 1024, 256
    wq = rng.integers(0, 0x7F, (N, K), dtype=np.uint8)
    wq[rng.random((N, K)) < 0.5] |= 0x80
    sb = (rng.uniform(0.5, 2.0, (N, K // 128)) * 0.01).astype(np.float32)  # not bf16 values
    deq = codecs.bf16_round(codecs.e4m3_decode(wq) * np.repeat(codecs.bf16_round(sb), 128, axis=1))
    for M in (16, 256):
        ks = (np.arange(M) * (K // M) + np.arange(M) * 3) % K
        x = np.zeros((M, K), np.float32)
        x[np.arange(M), ks] = 1.0
        y = ops.gemm(_capi.W8A16_BLK, _t(x, dev, torch.bfloat16), _t(wq, dev), w_scale=_t(sb, dev), ws_bn=1)
        np.testing.assert_array_equal(y.float().cpu().numpy(), deq[:, ks].T)
