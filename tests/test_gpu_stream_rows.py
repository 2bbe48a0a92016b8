"""Dense problems of a few dozen rows on the streaming kernel in 16-row
slices (`qmoe_gemm_plan` path "stream_rows"): every slice's workgroups
stream the whole weight matrix, one slice per grid.z index.

A slice computes exactly what the streaming kernel computes for those 16
rows alone (same kernel, same K walk), so the outputs are compared bit for
bit with per-slice calls where those plan the same kernel, and with the
oracle on sampled rows (`kernels/megablox/gmm_v2.py:452-462` W4A16,
`kernels/quantized_matmul/util.py:80-124` W8A8)."""

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


def _rows(M):
    return np.unique(np.linspace(0, M - 1, min(M, 7)).round().astype(np.int64))


@pytest.mark.parametrize("M", [17, 40, 64])
def test_mxfp4_slices_equal_single_slice_calls(dev, M):
    from qmoe import _capi, ops

    print(f"stream_rows mxfp4 M={M}", flush=True)
    K, N = 2880, 5760
    rng = np.random.default_rng(M)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = (127 + rng.integers(-8, 1, (N, K // 32))).astype(np.uint8)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xt, wt, st = _t(x, dev, torch.bfloat16), _t(packed, dev), _t(sc, dev)
    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W4A16_MX, xt, wt, w_scale=st)
    assert plans[0][4] == "stream_rows", plans
    for r0 in range(0, M, 16):
        with ops.record_plans() as p1:
            ys = ops.gemm(_capi.W4A16_MX, xt[r0:r0 + 16].contiguous(), wt, w_scale=st)
        assert p1[0][4:] == ("stream", 16, 1), p1
        assert torch.equal(y[r0:r0 + 16].view(torch.int16), ys.view(torch.int16)), f"slice at row {r0}"
    r = _rows(M)
    ref = linear.w4a16_mxfp4(x[r], packed, sc)
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"mxfp4 rows M={M}")


@pytest.mark.parametrize("M", [20, 48])
def test_nvfp4_slices_with_fused_silu_and_bias(dev, M):
    from qmoe import _capi, ops

    print(f"stream_rows nvfp4 silu M={M}", flush=True)
    K, N = 1024, 768
    rng = np.random.default_rng(M + 1)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    blk = codecs.e4m3_decode(rng.integers(0x20, 0x48, (N, K // 16)).astype(np.uint8))
    sc = codecs.nvfp4_fuse_scales(blk, np.float32(0.0123456789))
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W4A16_NV, _t(x, dev, torch.bfloat16), _t(packed, dev),
                     w_scale=_t(sc, dev, torch.bfloat16), bias=_t(bias, dev), activation="silu")
    assert plans[0][4] == "stream_rows", plans
    # f32 gate / up sums (bias added), the activation, one bf16 rounding
    gu = (x.astype(np.float64) @ codecs.dequant_nvfp4(packed, sc).astype(np.float64).T).astype(np.float32)
    gu = (gu + bias[None, :]).astype(np.float32)
    ref = codecs.bf16_round(omoe.act_fn(gu[:, : N // 2], gu[:, N // 2:], "silu"))
    assert_close_rows(y.float().cpu().numpy(), ref, f"nvfp4 silu M={M}")


def test_fp8_down_projection_32_rows(dev):
    """The Llama-3-8B down projection (K 14336, N 4096) at 32 rows: two
    16-row slices of 128 tiles instead of one 32-row pass with a K split."""
    from qmoe import _capi, ops

    print("stream_rows fp8 down M=32", flush=True)
    M, K, N = 32, 14336, 4096
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq, dev), a_scale=xs, w_scale=_t(ws, dev))
    assert plans[0][4:] == ("stream_rows", 16, 1), plans
    assert ops.plan_for_shape(_capi.W8A8_PC, M, 14336, 4096)[4] != "stream_rows"  # the up projection
    r = _rows(M)
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, "fp8")
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, "fp8 down M=32")
