"""The hot-path ops are torch custom ops with fake implementations: shapes
and dtypes under FakeTensorMode (CPU, no kernel runs), a whole-graph trace
through them, and (GPU) torch.compile(fullgraph=True) against eager."""

import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from qmoe.layers.fused_moe import fused_moe_gmm
from qmoe.layers.linear_common import quantized_matmul, quantized_matmul_fp4
from qmoe.layers.moe_routing import rowmax_select, select_experts

E, H, I, T, K_TOP = 16, 256, 128, 15, 4


def _moe_weights(dev, fmt):
    if fmt == "nvfp4":
        return (torch.empty((E, 2 * I, H // 2), dtype=torch.uint8, device=dev),
                torch.empty((E, H, I // 2), dtype=torch.uint8, device=dev),
                torch.empty((E, 2 * I, H // 16), dtype=torch.bfloat16, device=dev),
                torch.empty((E, H, I // 16), dtype=torch.bfloat16, device=dev))
    if fmt == "int4":
        return (torch.empty((E, 2 * I, H // 8), dtype=torch.int32, device=dev),
                torch.empty((E, H, I // 8), dtype=torch.int32, device=dev),
                torch.empty((E, 2 * I, H // 64), dtype=torch.bfloat16, device=dev),
                torch.empty((E, H, I // 64), dtype=torch.bfloat16, device=dev))
    if fmt == "mxfp4":
        return (torch.empty((E, 2 * I, H // 2), dtype=torch.uint8, device=dev),
                torch.empty((E, H, I // 2), dtype=torch.uint8, device=dev),
                torch.empty((E, 2 * I, H // 32), dtype=torch.uint8, device=dev),
                torch.empty((E, H, I // 32), dtype=torch.uint8, device=dev))
    return (torch.empty((E, 2 * I, H), dtype=torch.float8_e4m3fn, device=dev),
            torch.empty((E, H, I), dtype=torch.float8_e4m3fn, device=dev),
            torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32, device=dev),
            torch.empty((E, H // 128, I // 128), dtype=torch.float32, device=dev))


def test_fake_shapes_and_dtypes():
    with FakeTensorMode():
        x = torch.empty((3, 5, 256), dtype=torch.bfloat16, device="cuda")
        w = torch.empty((384, 256), dtype=torch.float8_e4m3fn, device="cuda")
        y = quantized_matmul(x, w.t(), torch.empty((384,), device="cuda"))
        assert y.shape == (3, 5, 384) and y.dtype == torch.bfloat16
        y = quantized_matmul(x, w.t(), torch.empty((1, 2, 1, 384), device="cuda"))
        assert y.shape == (3, 5, 384)
        y = quantized_matmul_fp4(x, torch.empty((384, 128), dtype=torch.uint8, device="cuda"),
                                 torch.empty((384, 8), dtype=torch.uint8, device="cuda"))
        assert y.shape == (3, 5, 384)
        # NVFP4: bf16 (or f32) scales per 16 k
        y = quantized_matmul_fp4(x, torch.empty((384, 128), dtype=torch.uint8, device="cuda"),
                                 torch.empty((384, 16), dtype=torch.bfloat16, device="cuda"))
        assert y.shape == (3, 5, 384) and y.dtype == torch.bfloat16
        with pytest.raises(ValueError, match="NVFP4 weight"):
            quantized_matmul_fp4(x, torch.empty((384, 128), dtype=torch.uint8, device="cuda"),
                                 torch.empty((384, 8), dtype=torch.float32, device="cuda"))
        logits = torch.empty((T, E), dtype=torch.bfloat16, device="cuda")
        h = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        tw, ids = select_experts(h, logits, topk=K_TOP, renormalize=True, scoring_fn="softmax")
        assert tw.shape == (T, K_TOP) and tw.dtype == torch.bfloat16 and ids.dtype == torch.int32
        v, i = rowmax_select(torch.empty((7, E), device="cuda"), 3)
        assert v.shape == (7, 3) and v.dtype == torch.float32 and i.dtype == torch.int32
        for fmt in ("mxfp4", "fp8_block", "nvfp4", "int4"):
            w1, w2, s1, s2 = _moe_weights("cuda", fmt)
            out = fused_moe_gmm(h, w1, w2, s1, s2, None, None, tw, ids, None, K_TOP, "silu", weight_format=fmt)
            assert out.shape == (T, H) and out.dtype == torch.bfloat16
        # the reference's int4 marker selects the packed-int4 format from int32 carriers
        w1, w2, s1, s2 = _moe_weights("cuda", "int4")
        out = fused_moe_gmm(h, w1, w2, s1, s2, None, None, tw, ids, None, K_TOP, "silu", rhs_quant_dtype="int4")
        assert out.shape == (T, H)
        with pytest.raises(NotImplementedError):
            fused_moe_gmm(h, w1, w2, s1, s2, None, None, tw, ids, None, K_TOP, "silu", rhs_quant_dtype="int2")


def test_layer_traces_as_one_graph_of_qmoe_ops():
    from torch.fx.experimental.proxy_tensor import make_fx

    def layer(h, logits, w1, w2, s1, s2, wl, sl):
        tw, ids = select_experts(h, logits, topk=K_TOP, renormalize=True, scoring_fn="softmax")
        y = fused_moe_gmm(h, w1, w2, s1, s2, None, None, tw, ids, None, K_TOP, "swigluoai", weight_format="mxfp4")
        return quantized_matmul(y, wl.t(), sl)

    with FakeTensorMode():
        args = (torch.empty((T, H), dtype=torch.bfloat16, device="cuda"),
                torch.empty((T, E), dtype=torch.bfloat16, device="cuda"),
                *_moe_weights("cuda", "mxfp4"),
                torch.empty((64, H), dtype=torch.float8_e4m3fn, device="cuda"),
                torch.empty((64,), device="cuda"))
        gm = make_fx(layer, tracing_mode="fake")(*args)
    targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    for op in ("qmoe.moe_route.default", "qmoe.fused_moe_gmm.default", "qmoe.quantized_matmul.default"):
        assert op in targets, (op, targets)


def test_checks_raise_before_the_op():
    with FakeTensorMode():
        x = torch.empty((2, 256), dtype=torch.bfloat16, device="cuda")
        w = torch.empty((384, 128), dtype=torch.float8_e4m3fn, device="cuda")
        with pytest.raises(ValueError, match="must match weight hidden dim"):
            quantized_matmul(x, w.t(), torch.empty((384,), device="cuda"))
        with pytest.raises(NotImplementedError):
            select_experts(x, torch.empty((2, 8), device="cuda"), topk=2, renormalize=True, scoring_fn="relu")


@pytest.mark.gpu
def test_compiled_fullgraph_matches_eager(dev):
    rng = np.random.default_rng(3)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    w1 = t(rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8))
    w2 = t(rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8))
    s1 = t((127 + rng.integers(-8, 1, (E, 2 * I, H // 32))).astype(np.uint8))
    s2 = t((127 + rng.integers(-8, 1, (E, H, I // 32))).astype(np.uint8))
    wl = (torch.randn((64, H), device=dev) * 0.02).to(torch.float8_e4m3fn)
    sl = torch.rand(64, device=dev) + 0.5
    h = torch.randn((T, H), device=dev).to(torch.bfloat16)
    logits = torch.randn((T, E), device=dev).to(torch.bfloat16)

    def layer(h, logits):
        tw, ids = select_experts(h, logits, topk=K_TOP, renormalize=True, scoring_fn="softmax")
        y = fused_moe_gmm(h, w1, w2, s1, s2, None, None, tw, ids, None, K_TOP, "swigluoai", weight_format="mxfp4")
        return quantized_matmul(y, wl.t(), sl)

    ref = layer(h, logits)
    got = torch.compile(layer, fullgraph=True, backend="aot_eager")(h, logits)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
