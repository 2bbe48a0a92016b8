"""The per-call scratch of `qmoe/ops.py` (split-K partial sums, the fused
decode op's dispatch and intermediates) under HIP graph capture and on
concurrent streams.

The scratch comes from torch's caching allocator on the current stream, so
a graph captured around a call keeps its own block for its lifetime
(a later, larger problem cannot free or move it), and two streams never
share bytes. The results are compared bit for bit with eager calls of the
same deterministic kernels (split-K slices and decode partials are summed in
a fixed order)."""

import ctypes

import numpy as np
import pytest
import torch

from test_gpu_decode import _layer, _run, _f8, _t as _td
from oracle import codecs, linear, quant

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


def _splitk_problem(dev, seed, M, N, K):
    """An FP8 W8A8 per-channel GEMM whose plan needs split-K scratch; returns
    (call, oracle output)."""
    from qmoe import _capi, ops

    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    ref, _, _ = linear.w8a8_per_channel(x, wq, ws, "fp8")
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    wt, wst = _t(wq, dev), _t(ws, dev)
    d, _ = ops.gemm_desc(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst)
    need = ctypes.c_int64(0)
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 0
    assert need.value > 0, f"M={M} N={N} K={K} plans no split-K scratch"

    def call(out=None):
        return ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, out=out)

    return call, ref, need.value


def test_graph_replays_after_a_larger_call(dev):
    """Capture a split-K GEMM and a fused decode step in one graph, then run
    eager calls that need far more scratch, then replay: every replay equals
    the eager result."""
    from qmoe import ops

    print("workspace: graph capture of split-K gemm + moe_decode, larger eager calls between replays", flush=True)
    small, _, need_small = _splitk_problem(dev, 1, 4, 1024, 14336)
    big, big_ref, need_big = _splitk_problem(dev, 2, 48, 4096, 14336)
    assert need_big > need_small
    L = _layer(11, 32, 1024, 512, 256, 5, 6)
    x = _td(L["hidden"], dev, torch.bfloat16)
    dec_args = (_f8(L["w1q"], dev), _f8(L["w2q"], dev), _td(L["w1s"], dev), _td(L["w2s"], dev),
                _f8(L["shared_w1q"], dev), _td(L["shared_w1s"], dev), _f8(L["shared_w2q"], dev),
                _td(L["shared_w2s"], dev), _td(L["shared_gate"], dev, torch.bfloat16),
                _td(L["topk_weights"], dev, torch.bfloat16), _td(L["topk_ids"], dev))
    eager_gemm = small()
    eager_dec = _run(L, dev)
    g_out = torch.empty_like(eager_gemm)
    d_out = torch.empty((x.shape[0], x.shape[1]), dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        small(out=g_out)
        ops.moe_decode(x, *dec_args, out=d_out)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            small(out=g_out)
            ops.moe_decode(x, *dec_args, out=d_out)
    torch.cuda.synchronize()
    for rep in range(3):
        g_out.zero_()
        d_out.zero_()
        y = big()  # needs more scratch than the captured calls
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, eager_gemm), f"replay {rep}: split-K gemm differs from eager"
        np.testing.assert_array_equal(d_out.float().cpu().numpy(), eager_dec, err_msg=f"replay {rep}: decode")
        if rep == 0:
            from conftest import assert_close_same_codes

            assert_close_same_codes(y.float().cpu().numpy(), big_ref, "larger eager split-K gemm")
    del g


def test_concurrent_streams(dev):
    """Two streams run different split-K GEMMs back to back without
    synchronising with each other: each output equals its eager result."""
    print("workspace: two streams, split-K gemms interleaved", flush=True)
    a_call, _, _ = _splitk_problem(dev, 3, 4, 2048, 14336)
    b_call, _, _ = _splitk_problem(dev, 4, 6, 1024, 14336)
    a_ref, b_ref = a_call(), b_call()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs_a, outs_b = [], []
    for _ in range(8):
        with torch.cuda.stream(s1):
            outs_a.append(a_call())
        with torch.cuda.stream(s2):
            outs_b.append(b_call())
    torch.cuda.synchronize()
    for o in outs_a:
        assert torch.equal(o, a_ref)
    for o in outs_b:
        assert torch.equal(o, b_ref)
