"""The allocation-free GEMM entry point `qmoe_gemm_static` (split-K partial
sums in the library's static device scratch) against `qmoe_gemm` with a
caller workspace: identical outputs (same kernels, same summation order) on
two calls in a row, the second smaller, for the streaming and the tiled
split-K paths; problems whose partials exceed the scratch are refused on the
host."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import codecs, quant

pytestmark = pytest.mark.gpu


def _lib():
    from qmoe import _capi

    return _capi.lib


def _case(dev, M, K, N, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    xq, xs = quant.quantize_act(x, "fp8")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return t(xq), t(xs), t(wq), t(ws)


def _static_gemm(lib, xq, xs, wq, ws, activation=None):
    """`qmoe_gemm_static` through the C ABI, output allocated by the caller."""
    from qmoe import _capi, ops

    M, N = xq.shape[0], wq.shape[0]
    out = torch.empty((M, N // 2 if activation else N), dtype=torch.bfloat16, device=xq.device)
    d, out = ops.gemm_desc(_capi.W8A8_PC, xq, wq, a_scale=xs, w_scale=ws, activation=activation, out=out)
    st = lib.qmoe_gemm_static(ctypes.byref(d), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st, out, ops.plan_of_desc(d)


@pytest.mark.parametrize("shapes,act", [
    # streaming kernel with a K split (decode rows, tall K), then fewer rows
    (((4, 14336, 1024), (2, 14336, 1024)), None),
    # 1-byte tiled kernel with a 4-way K split, then a smaller M
    (((96, 14336, 1024), (40, 14336, 1024)), None),
    # tiled split-K finishing kernel with a fused activation, then smaller
    (((100, 8192, 640), (33, 8192, 640)), "silu"),
])
def test_gemm_static_matches_gemm(dev, shapes, act):
    from qmoe import _capi, ops

    lib = _lib()
    for i, (M, K, N) in enumerate(shapes):
        print(f"gemm_static M={M} K={K} N={N} act={act}", flush=True)
        xq, xs, wq, ws = _case(dev, M, K, N, seed=M + K + N)
        a, w = xq.view(torch.uint8), wq.view(torch.uint8)
        st, got, plan = _static_gemm(lib, a, xs, w, ws, act)
        assert st == 0, _capi.STATUS_TEXT.get(st, st)
        assert plan[6] > 1, f"the case must use the scratch (K split), plan {plan}"
        ref = ops.gemm(_capi.W8A8_PC, a, w, a_scale=xs, w_scale=ws, activation=act)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"call {i}: static-scratch output differs"


def test_gemm_static_generic_k_split(dev):
    """The generic tiled kernel's K split (bf16 activations x bf16 weights,
    DeepSeek-V3's router gate shape) with its f32 slices in the static
    scratch: identical to qmoe_gemm on two calls in a row, the second
    smaller."""
    from qmoe import _capi, ops

    lib = _lib()
    K, N = 7168, 256
    rng = np.random.default_rng(7)
    w = torch.from_numpy(codecs.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))).to(dev)
    w = w.to(torch.bfloat16)
    for M in (4096, 1000):
        print(f"gemm_static generic K split M={M} K={K} N={N}", flush=True)
        x = torch.from_numpy(codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))).to(dev)
        x = x.to(torch.bfloat16)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        d, out = ops.gemm_desc(_capi.W16A16, x, w, out=out)
        plan = ops.plan_of_desc(d)
        assert plan[4] == "tiled_generic" and plan[6] > 1, plan
        st = lib.qmoe_gemm_static(ctypes.byref(d), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, _capi.STATUS_TEXT.get(st, st)
        ref = ops.gemm(_capi.W16A16, x, w)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"M={M}: static-scratch output differs"


def test_gemm_static_refuses_oversized_partials(dev):
    """A problem whose split-K partials exceed the scratch is refused before
    any launch (status QMOE_ERR_SCRATCH = 4)."""
    from qmoe import _capi, ops

    lib = _lib()
    cap = lib.qmoe_gemm_static_scratch_bytes()
    assert cap == 64 << 20
    # 256 tokens, K 14336, N 24576: 1-byte tiles with a 4-way split,
    # 4 * 256 * 24576 * 4 bytes = 96 MiB of partials
    M, K, N = 256, 14336, 24576
    plan = ops.plan_for_shape(_capi.W8A8_PC, M, N, K)
    assert plan[6] * M * N * 4 > cap, plan
    a = torch.zeros((M, K), dtype=torch.uint8, device=dev)
    s = torch.ones(M, dtype=torch.float32, device=dev)
    w = torch.zeros((N, K), dtype=torch.uint8, device=dev)
    ws = torch.ones(N, dtype=torch.float32, device=dev)
    st, _, _ = _static_gemm(lib, a, s, w, ws)
    assert st == 4


def test_gemm_static_mx_activations(dev):
    """The opt-in MX kind (QMOE_W4A4_MX, no K split, no scratch) through the
    allocation-free entry: bit-identical to `qmoe_gemm` on two calls in a
    row, the second smaller."""
    from qmoe import _capi, ops

    lib = _lib()
    for i, (M, N, K) in enumerate(((512, 1024, 2048), (200, 520, 1024))):
        print(f"gemm_static mx M={M} N={N} K={K}", flush=True)
        rng = np.random.default_rng(M + N)
        x = torch.from_numpy(codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))).to(dev)
        q, s = ops.mx_quant(x.to(torch.bfloat16))
        wq = torch.from_numpy(rng.integers(0, 256, (N, K // 2), dtype=np.uint8)).to(dev)
        ws = torch.from_numpy(rng.integers(118, 130, (N, K // 32), dtype=np.uint8)).to(dev)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        d, out = ops.gemm_desc(_capi.W4A4_MX, q, wq, a_scale=s, w_scale=ws, out=out)
        st = lib.qmoe_gemm_static(ctypes.byref(d), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, _capi.STATUS_TEXT.get(st, st)
        assert ops.plan_of_desc(d)[4] == "tiled_mx_persistent"
        ref = ops.gemm(_capi.W4A4_MX, q, wq, a_scale=s, w_scale=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: static output differs"
