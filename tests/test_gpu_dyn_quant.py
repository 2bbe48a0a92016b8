"""Per-channel W8A8 with the per-token activation quantization inside the
GEMM call (`QMOE_W8A8_PC_DYN`): the whole `xla_quantized_matmul` of
`kernels/quantized_matmul/util.py:80-124` (quantize_block `:294-318`, then
the W8A8 dot) in one C-ABI call.

Decode-size problems quantize inside the weight-streaming kernel; larger
ones quantize into the workspace and run the per-channel GEMM. Either way
the codes are the ones `qmoe_row_quant` (mode 0) writes and the MFMA
sequence is the two-launch path's, so the outputs are compared with that
path bit for bit (a NaN output's sign aside: for a product of two NaNs the
result's sign depends on the operand order the compiler picks), and with the
oracle on sampled rows.
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


_W = {}


def _weights(dev, qd, N, K):
    key = (qd, N, K)
    if key not in _W:
        _W.clear()
        rng = np.random.default_rng(N + K + (qd == "int8"))
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        wq, ws = quant.quantize_tensor(w, qd)
        _W[key] = (wq, ws, _t(wq.view(np.uint8), dev), _t(ws, dev))
    return _W[key]


def _two_launch(x, wt, wst, qd):
    from qmoe import _capi, ops

    xq, xs = ops.row_quant(x, qd)
    return ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=int(qd == "int8"))


def _dyn(x, wt, wst, qd):
    from qmoe import _capi, ops

    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W8A8_PC_DYN, x, wt, w_scale=wst, wfmt=int(qd == "int8"))
    return y, plans[0][4]


def _bits(t):
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 64, 300])
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096), (1024, 384)])
@pytest.mark.parametrize("qd", ["fp8", "int8"])
def test_dyn_matches_two_launch_path(dev, qd, K, N, M):
    print(f"w8a8 dyn {qd} K={K} N={N} M={M}", flush=True)
    wq, ws, wt, wst = _weights(dev, qd, N, K)
    rng = np.random.default_rng(M * 7 + K)
    x = codecs.bf16_round((rng.standard_normal((M, K)) * np.exp2(rng.integers(-6, 7, (M, 1)))).astype(np.float32))
    if M > 2:
        x[1] = 0.0  # a zero row: scale 1, codes 0
    xt = _t(x, dev, torch.bfloat16)
    y, path = _dyn(xt, wt, wst, qd)
    if M == 1:
        assert path == "stream_dyn", path
    np.testing.assert_array_equal(_bits(y), _bits(_two_launch(xt, wt, wst, qd)))
    r = np.unique(np.linspace(0, M - 1, min(M, 5)).round().astype(np.int64))
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, qd)
    got = y[torch.from_numpy(r).to(dev)].float().cpu().numpy()
    if qd == "int8":
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_same_codes(got, ref, f"dyn {qd} M={M}")


@pytest.mark.parametrize("M", [2, 3, 4, 16, 17, 32])
@pytest.mark.parametrize("qd", ["fp8", "int8"])
def test_dyn_in_kernel_rows(dev, monkeypatch, qd, M):
    """The in-kernel form beyond its default row limit (QMOE_DYN_FUSE_ROWS):
    several rows per workgroup's codes, and two 16-row M tiles per pass
    (rows 17-32)."""
    monkeypatch.setenv("QMOE_DYN_FUSE_ROWS", "32")
    print(f"w8a8 dyn two-tile pass {qd} M={M}", flush=True)
    K, N = 4096, 1024
    _, _, wt, wst = _weights(dev, qd, N, K)
    x = torch.randn((M, K), device=dev, generator=torch.Generator(device=dev).manual_seed(M)).to(torch.bfloat16)
    y, path = _dyn(x, wt, wst, qd)
    assert path == "stream_dyn"
    assert torch.equal(y.view(torch.int16), _two_launch(x, wt, wst, qd).view(torch.int16))


def _same_bits_nan_sign_aside(y, ref):
    """Bit-equal outputs, except that a NaN may carry either sign."""
    a, b = _bits(y), _bits(ref)
    nan_a = (a & 0x7F80) == 0x7F80
    nan_a &= (a & 0x7F) != 0
    nan_b = (b & 0x7F80) == 0x7F80
    nan_b &= (b & 0x7F) != 0
    np.testing.assert_array_equal(nan_a, nan_b)
    np.testing.assert_array_equal(np.where(nan_a, 0, a), np.where(nan_b, 0, b))


@pytest.mark.parametrize("qd", ["fp8", "int8"])
@pytest.mark.parametrize("M,K,N,fuse", [(4, 4096, 2048, "4"), (4, 14336, 1024, "4"),
                                        # the default row limit, both tile widths (N 384: two
                                        # 16-row weight tiles per workgroup)
                                        (2, 1024, 384, None), (2, 4096, 14336, None), (1, 4096, 14336, None)])
def test_dyn_non_finite_rows(dev, monkeypatch, qd, M, K, N, fuse):
    """Rows holding inf or NaN take the quantizer's exact slow path inside
    the kernel: the same bits as the two-launch path (a NaN's sign aside),
    and the finite rows are untouched."""
    if fuse:
        monkeypatch.setenv("QMOE_DYN_FUSE_ROWS", fuse)
    print(f"w8a8 dyn non-finite rows {qd} M={M} K={K} N={N}", flush=True)
    _, _, wt, wst = _weights(dev, qd, N, K)
    rng = np.random.default_rng(K + M)
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    if M == 4:
        x[1, 7] = np.inf
        x[2, K - 1] = np.nan
        x[3, 100] = -np.inf
    else:
        x[M - 1, K - 3] = np.nan
        x[0, 5] = np.inf
    xt = _t(x, dev, torch.bfloat16)
    y, path = _dyn(xt, wt, wst, qd)
    assert path == "stream_dyn"
    _same_bits_nan_sign_aside(y, _two_launch(xt, wt, wst, qd))
    if M == 4:
        assert torch.isfinite(y[0].float()).all()


def test_quantized_matmul_decode_is_one_launch(dev):
    """`quantized_matmul` per-channel W8A8 at decode size runs the fused
    path (the streaming kernel quantizing inside) and equals the two-launch
    result bit for bit."""
    from qmoe import ops
    from qmoe.layers.linear_common import quantized_matmul

    K, N = 4096, 14336
    _, _, wt, wst = _weights(dev, "fp8", N, K)
    x = torch.randn((1, K), device=dev).to(torch.bfloat16)
    w = wt.view(torch.float8_e4m3fn)
    with ops.record_plans() as plans:
        y = quantized_matmul(x, w.t(), wst)
    assert [p[4] for p in plans] == ["stream_dyn"]
    assert torch.equal(y.view(torch.int16), _two_launch(x, wt, wst, "fp8").view(torch.int16))
