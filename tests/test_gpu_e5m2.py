"""float8_e5m2 weight codes (`REQUANTIZE_WEIGHT_DTYPE` /
`MOE_REQUANTIZE_WEIGHT_DTYPE=float8_e5m2`, `layers/adapter/quantization/
fp8.py:122-127`) through the C-ABI.

* the quantizer (`qmoe_row_quant` qdtype 2): load-time and runtime codes and
  scales bit-exact against the oracle, whose e5m2 encoder is pinned to
  torch's float8_e5m2 cast; every e5m2 rounding boundary through the device
  encoders (the hardware conversion on rows with a finite scale, the
  software encoder on the others);
* per-channel W8A8 with e5m2 on both operands (`util.py:80-124` quantizes
  the activations to the weight dtype): the streaming, narrow-tile and
  256-wide tile kernels, with the quantization inside the call or before it;
* the grouped-matmul recipe with e5m2 weights and e4m3 activations
  (`kernels/megablox/gmm_v2.py:1199-1215`), per channel and per (row, 512).
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_same_codes
from oracle import codecs, linear, quant

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _boundaries():
    """Every finite e5m2 value, every midpoint between neighbours (exact
    ties) and the f32 neighbours of each midpoint, |x| <= 57344, both signs."""
    vals = codecs.e5m2_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    fin = np.unique(vals[np.isfinite(vals)])
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)
    x = np.concatenate([fin.astype(np.float32), mids, np.nextafter(mids, np.float32(1e9)),
                        np.nextafter(mids, np.float32(-1e9)), np.float32([-0.0, 2.0 ** -17, -(2.0 ** -17)])])
    return x[np.abs(x) <= 57344].astype(np.float32)


def test_e5m2_load_time_boundaries(dev):
    """Load-time rows (f32 in, reciprocal multiply): the row's absmax 57344
    makes the scale ~1, so the codes are the encoder's on each boundary."""
    from qmoe import ops

    print("row_quant e5m2 load boundaries", flush=True)
    x = _boundaries()
    n = (x.size + 127) // 128 * 128
    row = np.zeros(n, np.float32)
    row[: x.size] = x
    row[-1] = 57344.0
    rows = np.stack([row, row * np.float32(3.0), np.zeros(n, np.float32)])
    q_ref, s_ref = quant.quantize_tensor(rows, "e5m2")
    q, s = ops.row_quant(_t(rows, dev), "e5m2", mode="load")
    assert q.dtype == torch.float8_e5m2
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_e5m2_runtime_boundaries(dev):
    """Runtime rows (bf16 in, division): scale exactly 1 (absmax 57344) and
    57344 / 57344 * 3, on the bf16-representable boundary values; the
    hardware conversion of the fast path against the oracle's encoder."""
    from qmoe import ops

    print("row_quant e5m2 runtime boundaries", flush=True)
    x = np.unique(codecs.bf16_round(_boundaries()))
    n = (x.size + 127) // 128 * 128
    rows = np.zeros((2, n), np.float32)
    rows[0, : x.size] = x
    rows[0, -1] = 57344.0
    rows[1] = codecs.bf16_round(rows[0] * np.float32(3.0))
    q_ref, s_ref = quant.quantize_act(rows, "e5m2")
    q, s = ops.row_quant(_t(rows, dev, torch.bfloat16), "e5m2")
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))


@pytest.mark.parametrize("M,K", [(1, 4096), (7, 2048), (64, 7168), (3, 14336), (2, 40960), (600, 7168),
                                 (300, 14336)])
def test_e5m2_runtime_rows(dev, M, K):
    """Random rows across exponents, a zero row (scale 1), an outlier, and
    rows with inf / NaN (the software encoder's slow path): codes and scales
    bit-exact, except the sign of NaN codes (the sign of the NaN that inf /
    inf makes differs between the host's division and the device's)."""
    from qmoe import ops

    print(f"row_quant e5m2 M={M} K={K}", flush=True)
    rng = np.random.default_rng(M * 13 + K)
    x = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-20, 12, (M, 1)))).astype(np.float32)
    x[0, :] = 0.0
    if M > 2:
        x[2, 5] = 1e4
    if M > 4:
        x[3, 9] = np.inf
        x[4, 1] = np.nan
    x = codecs.bf16_round(x)
    q_ref, s_ref = quant.quantize_act(x, "e5m2")
    q, s = ops.row_quant(_t(x, dev, torch.bfloat16), "e5m2")
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    got, ref = q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8)
    nan = (ref & 0x7F) == 0x7F
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    assert ((got[nan] & 0x7F) == 0x7F).all()
    assert nan.any() == (M > 4)


_W = {}


def _weights(dev, N, K):
    key = (N, K)
    if key not in _W:
        _W.clear()
        rng = np.random.default_rng(N + 3 * K)
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        wq, ws = quant.quantize_tensor(w, "e5m2")
        _W[key] = (wq, ws, _t(wq, dev), _t(ws, dev))
    return _W[key]


# decode (streaming, in-kernel quantization at M=1), mid-M (narrow tiles)
# and large M (256-wide tiles)
@pytest.mark.parametrize("M,K,N", [(1, 4096, 14336), (1, 14336, 4096), (5, 4096, 2048), (64, 4096, 14336),
                                   (256, 2048, 2048), (1024, 4096, 4096)])
def test_e5m2_per_channel_w8a8(dev, M, K, N):
    from qmoe import _capi, ops

    print(f"w8a8 e5m2 per channel M={M} K={K} N={N}", flush=True)
    wq, ws, wt, wst = _weights(dev, N, K)
    rng = np.random.default_rng(M + K)
    x = codecs.bf16_round((rng.standard_normal((M, K)) * np.exp2(rng.integers(-4, 5, (M, 1)))).astype(np.float32))
    xt = _t(x, dev, torch.bfloat16)
    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W8A8_PC_DYN, xt, wt, w_scale=wst, wfmt=2)
    print(f"  plan {plans[0][4]}", flush=True)
    xq, xs = ops.row_quant(xt, "e5m2")
    y2 = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=2)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    r = np.unique(np.linspace(0, M - 1, min(M, 6)).round().astype(np.int64))
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, "e5m2")
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"e5m2 pc M={M}")


@pytest.mark.parametrize("B", [None, 512])
@pytest.mark.parametrize("M,K,N", [(1, 2048, 1024), (16, 4096, 2048), (300, 2048, 1536), (1024, 4096, 4096)])
def test_e5m2_weights_gmm_recipe(dev, M, K, N, B):
    """`quantized_matmul` with a rank-4 scale over e5m2 weights: e4m3
    activations per (token, 512), e5m2 weights per channel (B = K) or per
    (row, 512)."""
    from qmoe.layers.linear_common import quantized_matmul

    print(f"gmm recipe e5m2 weights M={M} K={K} N={N} B={B}", flush=True)
    rng = np.random.default_rng(M * 3 + K + N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, wsb = quant.quantize_tensor(w, "e5m2", block=B or K)
    wsb = wsb.reshape(N, -1)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    wt = _t(wq, dev).view(torch.float8_e5m2)
    s4 = _t(np.ascontiguousarray(wsb.T), dev)[None, :, None, :]
    y = quantized_matmul(_t(x, dev, torch.bfloat16), wt.t(), s4)
    r = np.unique(np.linspace(0, M - 1, min(M, 6)).round().astype(np.int64))
    ref, _, _ = linear.w8a8_gmm(x[r], wq, wsb if B else wsb[:, 0], "fp8", wdtype="e5m2")
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"e5m2 gmm M={M} B={B}")
