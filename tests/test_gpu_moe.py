"""GPU parity of the MoE path: router (ids bit-exact), dispatch (bit-exact),
combine, and the whole fused layer for each weight format."""

import numpy as np
import pytest
import torch

from conftest import assert_close_rows
from oracle import codecs, moe as omoe, quant, routing

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(dtype) if dtype is not None else t


@pytest.mark.parametrize("T,E,k", [(1, 128, 4), (37, 128, 4), (1000, 256, 8), (64, 512, 10)])
def test_route_softmax_renorm(dev, T, E, k):
    from qmoe import ops

    print(f"route softmax T={T} E={E} k={k}", flush=True)
    rng = np.random.default_rng(T + E)
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    if T > 3:
        logits[1, :] = 0.0                  # all tied -> ids 0..k-1
        logits[2, 10:20] = 5.0              # tie across the k boundary
        logits[3, :] = np.nan               # poisoned row
    w_ref, ids_ref = routing.select_experts(logits, k, True, "softmax")
    w, ids = ops.moe_route(_t(logits, dev, torch.bfloat16), k, "softmax", True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    wg = w.float().cpu().numpy()
    np.testing.assert_array_equal(np.isnan(wg), np.isnan(w_ref))
    ok = ~np.isnan(w_ref)
    np.testing.assert_allclose(wg[ok], w_ref[ok], rtol=8e-3, atol=1e-6)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("T", [1, 8, 513])
def test_route_sigmoid_bias(dev, grouped, T):
    """DeepSeek-V3 routing: sigmoid, correction bias, (grouped) top-8,
    renormalize, routed_scaling_factor 2.5."""
    from qmoe import ops

    print(f"route sigmoid grouped={grouped} T={T}", flush=True)
    E, k = 256, 8
    rng = np.random.default_rng(T * 3 + grouped)
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    if grouped:
        w_ref, ids_ref = routing.grouped_topk(logits, k, True, 8, 4, "sigmoid", bias, 2.5)
    else:
        w_ref, ids_ref = routing.select_experts(logits, k, True, "sigmoid", bias, 2.5)
    w, ids = ops.moe_route(_t(logits, dev, torch.bfloat16), k, "sigmoid", True, bias=_t(bias, dev),
                           routed_scaling_factor=2.5, num_expert_group=8 if grouped else 1,
                           topk_group=4 if grouped else 1)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.float().cpu().numpy(), w_ref, rtol=8e-3, atol=1e-6)


@pytest.mark.parametrize("T,E,k,scoring,ng,tg,use_bias", [
    (7, 512, 8, "sigmoid", 8, 3, True),        # groups of 64 (one slot each)
    (9, 384, 8, "sigmoid", 6, 2, True),        # groups of 64, 6 of 8 slots hold experts
    (1, 256, 8, "sigmoid", 32, 8, True),       # groups of 8
    (5, 128, 8, "sigmoid", 64, 16, True),      # groups of 2
    (6, 128, 4, "softmax", 32, 4, False),      # groups of 4, group score = max
    (4, 64, 6, "softmax", 64, 20, False),      # groups of 1
    (5, 160, 6, "softmax", 8, 3, False),       # groups of 20 (not a power of two)
    (6, 96, 6, "sqrtsoftplus", 6, 3, True),    # groups of 16, half of slot 1 empty
])
@pytest.mark.parametrize("ties", [False, True])
def test_route_grouped_group_sizes(dev, T, E, k, scoring, ng, tg, use_bias, ties):
    """Grouped routing for every group-size regime of the kernel (DPP within a
    row, row broadcasts for 32 / 64, the LDS loop otherwise), against the
    oracle; `ties` draws logits and bias from a coarse grid so that choice and
    group scores tie exactly (lowest expert / group wins)."""
    from qmoe import ops

    print(f"route grouped T={T} E={E} k={k} {scoring} groups=({ng},{tg}) bias={use_bias} ties={ties}", flush=True)
    rng = np.random.default_rng(T * 7 + E + ng + ties)
    if ties:
        logits = (rng.integers(-4, 5, (T, E)) * 0.25).astype(np.float32)
        bias = (rng.integers(-2, 3, E) * 0.125).astype(np.float32) if use_bias else None
    else:
        logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
        bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if use_bias else None
    rsf = 2.5 if use_bias else 1.0
    w_ref, ids_ref = routing.grouped_topk(logits, k, True, ng, tg, scoring, bias, rsf)
    w, ids = ops.moe_route(_t(logits, dev, torch.bfloat16), k, scoring, True,
                           bias=_t(bias, dev) if bias is not None else None, routed_scaling_factor=rsf,
                           num_expert_group=ng, topk_group=tg)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.float().cpu().numpy(), w_ref, rtol=8e-3, atol=1e-6)
    if T * k <= 64 and T <= 16:
        w2, ids2, _ = ops.moe_route_dispatch(_t(logits, dev, torch.bfloat16), k, scoring, True,
                                             bias=_t(bias, dev) if bias is not None else None,
                                             routed_scaling_factor=rsf, num_expert_group=ng, topk_group=tg)
        np.testing.assert_array_equal(ids2.cpu().numpy(), ids_ref)
        np.testing.assert_array_equal(w2.view(torch.int16).cpu().numpy(), w.view(torch.int16).cpu().numpy())


@pytest.mark.parametrize("scoring,use_bias", [("sigmoid", True), ("softmax", False)])
def test_route_plain_ties(dev, scoring, use_bias):
    """Plain top-k with exact ties across and inside slots: lowest id first."""
    from qmoe import ops

    print(f"route plain ties {scoring}", flush=True)
    rng = np.random.default_rng(11)
    T, E, k = 12, 320, 8
    logits = (rng.integers(-3, 4, (T, E)) * 0.5).astype(np.float32)
    bias = (rng.integers(-1, 2, E) * 0.25).astype(np.float32) if use_bias else None
    w_ref, ids_ref = routing.select_experts(logits, k, True, scoring, bias, 1.0)
    w, ids = ops.moe_route(_t(logits, dev, torch.bfloat16), k, scoring, True,
                           bias=_t(bias, dev) if bias is not None else None)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.float().cpu().numpy(), w_ref, rtol=8e-3, atol=1e-6)


def test_rowmax_select_nan_and_sentinel_rows(dev):
    # tests/kernels/test_router_topk.py:101-135 (NaN, -inf, -FLT_MAX rows)
    from qmoe.layers.moe_routing import rowmax_select

    E, k = 512, 10
    for bad in (np.nan, -np.inf, np.finfo(np.float32).min):
        s = np.full((3, E), bad, np.float32)
        v, i = rowmax_select(_t(s, dev), k)
        assert np.isnan(v.cpu().numpy()).all()
        for row in i.cpu().numpy():
            assert sorted(row.tolist()) == list(range(k))
    rng = np.random.default_rng(5)
    s = rng.random((37, E), dtype=np.float32)
    s[:, :5] = np.nan
    v, i = rowmax_select(_t(s, dev), k)
    ref_v, ref_i = routing.rowmax_topk(s, k)
    np.testing.assert_array_equal(i.cpu().numpy(), ref_i)
    np.testing.assert_array_equal(v.cpu().numpy(), ref_v)


# from 8192 routes the chunked three-launch form runs: (2048, 4, 512) is
# exactly 8 chunks at the widest bucket row, (3001, 4, 128) has a ragged last
# chunk of 1764 routes, (2047, 4, 16) stays on the one-workgroup kernel
@pytest.mark.parametrize("T,k,E", [(3, 2, 2), (1, 8, 256), (64, 8, 256), (4096, 8, 256),
                                   (8192, 4, 128), (100, 10, 512), (2048, 4, 512), (3001, 4, 128),
                                   (2047, 4, 16)])
@pytest.mark.parametrize("skip_padded", [False, True])
def test_dispatch_bit_exact(dev, T, k, E, skip_padded):
    from qmoe import ops

    print(f"dispatch T={T} k={k} E={E} skip={skip_padded}", flush=True)
    rng = np.random.default_rng(T + k + E)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = codecs.bf16_round(rng.random((T, k)).astype(np.float32))
    if T >= 3:
        ids[1, -1] = -1
        w[2, :] = 0.0
    if T == 3 and k == 2:  # test_fused_moe_gmm.py:430-467 known answer
        ids = np.array([[1, 0], [0, -1], [1, 0]], np.int32)
        w = codecs.bf16_round(np.float32([[0.1, 0.2], [0.3, 0.0], [0.4, 0.5]]))
    ref = omoe.prepare_routed(ids, w, E, skip_padded)
    meta = ops.moe_dispatch(_t(ids, dev), _t(w, dev, torch.bfloat16), E, skip_padded)
    np.testing.assert_array_equal(meta["sorted_idx"].cpu().numpy(), ref["sorted_idx"])
    np.testing.assert_array_equal(meta["revert"].cpu().numpy(), ref["revert"])
    np.testing.assert_array_equal(meta["token_sorted"].cpu().numpy(), ref["token_sorted"])
    offs = meta["group_offs"].cpu().numpy()
    np.testing.assert_array_equal(np.diff(offs), ref["group_sizes"])
    na = int(meta["num_active"].cpu().item())
    np.testing.assert_array_equal(meta["active"].cpu().numpy()[:na], np.nonzero(ref["group_sizes"])[0])
    if T == 3 and k == 2 and not skip_padded:
        np.testing.assert_array_equal(ref["group_sizes"], [3, 2])


def _moe_case(fmt, E, k, H, I, T, seed, bias=False):
    rng = np.random.default_rng(seed)
    if fmt == "mxfp4":
        w13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
        s13 = (127 + rng.integers(-8, 1, (E, 2 * I, H // 32))).astype(np.uint8)
        w2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
        s2 = (127 + rng.integers(-8, 1, (E, H, I // 32))).astype(np.uint8)
    elif fmt == "nvfp4":
        # fused block scales: e4m3 block scale x a float32 global per expert (gate / up halves)
        w13 = rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8)
        w2 = rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8)
        b13s = rng.integers(0x20, 0x40, (E, 2 * I, H // 16)).astype(np.uint8)
        b2s = rng.integers(0x20, 0x40, (E, H, I // 16)).astype(np.uint8)
        s13 = codecs.nvfp4_fuse_scales(b13s, (rng.random((E, 2)) * 0.01 + 0.003).astype(np.float32), halves=True)
        s2 = codecs.nvfp4_fuse_scales(b2s, (rng.random(E) * 0.01 + 0.003).astype(np.float32))
    elif fmt.startswith("int4"):  # "int4-<group>": int32 carriers + bf16-valued group scales
        g = int(fmt.split("-")[1])
        w13 = codecs.int4_pack(rng.integers(-8, 8, (E, 2 * I, H)))
        w2 = codecs.int4_pack(rng.integers(-8, 8, (E, H, I)))
        s13 = codecs.bf16_round((rng.random((E, 2 * I, H // g)) * 0.004 + 0.001).astype(np.float32))
        s2 = codecs.bf16_round((rng.random((E, H, I // g)) * 0.004 + 0.001).astype(np.float32))
    elif fmt in ("fp8", "int8", "fp8_rowquant", "int8_rowquant", "fp8_w8a16"):
        qd = "int8" if fmt.startswith("int8") else "fp8"
        blk = 128 if fmt == "fp8_w8a16" else None
        r13 = [quant.quantize_tensor((rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32), qd, block=blk)
               for _ in range(E)]
        r2 = [quant.quantize_tensor((rng.standard_normal((H, I)) * 0.02).astype(np.float32), qd, block=blk)
              for _ in range(E)]
        w13, s13 = np.stack([q[0] for q in r13]), np.stack([q[1] for q in r13])
        w2, s2 = np.stack([q[0] for q in r2]), np.stack([q[1] for q in r2])
    elif fmt == "fp8_block":
        w13f = (rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32)
        w2f = (rng.standard_normal((E, H, I)) * 0.02).astype(np.float32)
        q13 = [quant.quantize_fp8_tiles(w13f[e]) for e in range(E)]
        q2 = [quant.quantize_fp8_tiles(w2f[e]) for e in range(E)]
        w13, s13 = np.stack([q[0] for q in q13]), np.stack([q[1] for q in q13])
        w2, s2 = np.stack([q[0] for q in q2]), np.stack([q[1] for q in q2])
    else:  # bf16
        w13 = codecs.bf16_round((rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32))
        w2 = codecs.bf16_round((rng.standard_normal((E, H, I)) * 0.05).astype(np.float32))
        s13 = s2 = None
    b13 = (rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32) if bias else None
    b2 = (rng.standard_normal((E, H)) * 0.1).astype(np.float32) if bias else None
    hid = codecs.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tw = codecs.bf16_round(rng.random((T, k)).astype(np.float32))
    return w13, s13, w2, s2, b13, b2, hid, ids, tw


@pytest.mark.parametrize("fmt,act,E,k,H,I,T,bias", [
    ("mxfp4", "swigluoai", 8, 2, 256, 256, 1, False),
    ("mxfp4", "swigluoai", 16, 4, 512, 384, 40, True),
    ("mxfp4", "swigluoai", 16, 4, 512, 256, 300, True),   # tiled path (T > 64)
    ("mxfp4", "swigluoai", 8, 2, 288, 160, 6, False),     # K % 256 != 0 in both GEMMs
    ("nvfp4", "silu", 8, 2, 256, 256, 1, False),
    ("nvfp4", "silu", 16, 4, 512, 384, 40, False),
    ("nvfp4", "gelu_tanh", 16, 4, 512, 256, 300, False),  # tiled path
    ("nvfp4", "silu", 8, 2, 288, 160, 6, False),          # K % 64 == 32 in both GEMMs
    ("int4-32", "silu", 8, 2, 256, 256, 1, False),
    ("int4-128", "silu", 16, 4, 512, 384, 40, False),
    ("int4-64", "silu", 16, 4, 512, 256, 300, False),      # tiled path
    ("int4-32", "silu", 8, 2, 288, 160, 6, False),         # K % 64 == 32 in both GEMMs
    ("fp8_block", "silu", 8, 2, 512, 256, 5, False),
    ("fp8_block", "silu", 16, 4, 512, 256, 200, False),   # tiled path
    ("fp8_block", "silu", 16, 4, 512, 256, 24, False),    # 6 rows per expert: tiled, 32-token tiles
    ("bf16", "silu", 8, 2, 256, 128, 9, False),
    ("bf16", "gelu_tanh", 8, 3, 256, 128, 100, True),
    # the grouped matmul's quantized-lhs recipe (per-channel experts)
    ("fp8", "silu", 8, 2, 1024, 256, 5, False),
    ("fp8", "silu", 16, 4, 1024, 384, 40, False),
    ("fp8", "swigluoai", 16, 4, 1024, 256, 300, True),    # tiled path
    ("int8", "silu", 8, 2, 1024, 256, 5, False),
    ("int8", "silu", 16, 4, 1024, 256, 300, False),       # tiled (generic) path
    ("fp8_w8a16", "silu", 8, 2, 512, 256, 5, False),
    ("fp8_w8a16", "silu", 16, 4, 512, 256, 300, True),
    ("fp8_rowquant", "silu", 16, 4, 512, 256, 40, False),
    ("int8_rowquant", "silu", 16, 4, 512, 256, 200, False),
])
def test_fused_moe_layer(dev, fmt, act, E, k, H, I, T, bias):
    from qmoe.layers.fused_moe import fused_moe_gmm

    print(f"fused moe {fmt} {act} E={E} k={k} H={H} I={I} T={T} bias={bias}", flush=True)
    w13, s13, w2, s2, b13, b2, hid, ids, tw = _moe_case(fmt, E, k, H, I, T, seed=E + T + H)
    ofmt = "int4" if fmt.startswith("int4") else fmt
    ref, _, _ = omoe.fused_moe(hid, omoe.ExpertWeights(ofmt, w13, s13, w2, s2, b13, b2), tw, ids, act)
    fp8_fmts = ("fp8_block", "fp8", "fp8_rowquant", "fp8_w8a16")
    wdt = torch.float8_e4m3fn if fmt in fp8_fmts else (torch.bfloat16 if fmt == "bf16" else None)

    def wt(a):
        t = _t(a, dev)
        if wdt is torch.float8_e4m3fn:
            return t.view(torch.float8_e4m3fn)
        return t.to(wdt) if wdt is not None else t

    sdt = torch.bfloat16 if fmt == "nvfp4" or ofmt == "int4" else None  # NVFP4 / INT4 runtime scales: bf16
    got = fused_moe_gmm(
        _t(hid, dev, torch.bfloat16), wt(w13), wt(w2),
        _t(s13, dev, sdt) if s13 is not None else None, _t(s2, dev, sdt) if s2 is not None else None,
        _t(b13, dev) if b13 is not None else None, _t(b2, dev) if b2 is not None else None,
        _t(tw, dev, torch.bfloat16), _t(ids, dev), None, k, act,
        weight_format=ofmt,
    )
    assert_close_rows(got.float().cpu().numpy(), ref, f"moe {fmt}")


@pytest.mark.parametrize("T,E,k,scoring,grouped,skip", [
    (1, 128, 4, "softmax", None, False), (5, 128, 4, "softmax", None, True), (16, 128, 4, "softmax", None, False),
    (1, 256, 8, "sigmoid", (8, 4), False), (8, 256, 8, "sigmoid", (8, 4), True), (3, 96, 6, "sigmoid", (6, 3), False),
    (16, 512, 4, "sqrtsoftplus", None, False), (2, 60, 5, "sigmoid", (5, 2), False)])
def test_route_dispatch_fused_matches_separate(dev, T, E, k, scoring, grouped, skip):
    """The decode launch that routes and dispatches in one workgroup gives
    exactly the outputs of the two separate entry points (and the oracle's
    permutation)."""
    from qmoe import ops

    print(f"route+dispatch T={T} E={E} k={k} {scoring} grouped={grouped} skip={skip}", flush=True)
    rng = np.random.default_rng(T * 31 + E + k)
    logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
    bias = _t((rng.standard_normal(E) * 0.1).astype(np.float32), dev) if scoring == "sigmoid" else None
    ng, tg = grouped if grouped else (1, 1)
    lt = _t(logits, dev, torch.bfloat16)
    kw = dict(bias=bias, routed_scaling_factor=2.5 if scoring == "sigmoid" else 1.0, num_expert_group=ng,
              topk_group=tg)
    w_ref, ids_ref = ops.moe_route(lt, k, scoring, True, **kw)
    meta_ref = ops.moe_dispatch(ids_ref, w_ref, E, skip)
    w, ids, meta = ops.moe_route_dispatch(lt, k, scoring, True, skip_padded_tokens=skip, **kw)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref.cpu().numpy())
    np.testing.assert_array_equal(w.view(torch.int16).cpu().numpy(), w_ref.view(torch.int16).cpu().numpy())
    for key in ("sorted_idx", "revert", "token_sorted", "group_offs", "num_active"):
        np.testing.assert_array_equal(meta[key].cpu().numpy(), meta_ref[key].cpu().numpy(), err_msg=key)
    na = int(meta["num_active"].item())
    np.testing.assert_array_equal(meta["active"][:na].cpu().numpy(), meta_ref["active"][:na].cpu().numpy())
    np.testing.assert_array_equal(meta["sorted_weight"].view(torch.int16).cpu().numpy(),
                                  meta_ref["sorted_weight"].view(torch.int16).cpu().numpy())
    p = omoe.prepare_routed(ids.cpu().numpy(), w.float().cpu().numpy(), E, skip)
    np.testing.assert_array_equal(meta["sorted_idx"].cpu().numpy(), p["sorted_idx"])
    np.testing.assert_array_equal(np.diff(meta["group_offs"].cpu().numpy()), p["group_sizes"])


def test_route_dispatch_rejects_large_batches(dev):
    from qmoe import ops

    logits = torch.zeros((17, 64), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.moe_route_dispatch(logits, 2, "softmax", True)
    with pytest.raises(ValueError):
        ops.moe_route_dispatch(logits[:9], 8, "softmax", True)


@pytest.mark.parametrize("scoring,E,k,T,renorm", [("softmax", 4, 2, 2, False), ("sigmoid", 256, 8, 37, True),
                                                  ("sqrtsoftplus", 384, 6, 5, True)])
def test_route_hash_table(dev, scoring, E, k, T, renorm):
    """DeepSeek-V4 hash routing through select_experts: ids bit-exact, weights
    vs the oracle; the reference known answer for the first case
    (`tests/layers/adapter/test_moe_routing.py:237-251`)."""
    from types import SimpleNamespace

    from qmoe.layers.moe_routing import select_experts

    print(f"route hash {scoring} E={E} k={k} T={T}", flush=True)
    rng = np.random.default_rng(E + T)
    if E == 4:
        logits = np.zeros((T, E), np.float32)
        table = np.array([[0, 1], [2, 3]], np.int32)
        inp = np.array([1, 0])
    else:
        logits = codecs.bf16_round(rng.standard_normal((T, E)).astype(np.float32))
        table = rng.integers(0, E, (100, k)).astype(np.int32)
        inp = rng.integers(0, 100, T)
    layer = SimpleNamespace(hash_indices_table=_t(table, dev), routed_scaling_factor=2.0,
                            e_score_correction_bias=None, use_grouped_topk=False)
    h = torch.zeros((T, 8), device=dev, dtype=torch.bfloat16)
    w, ids = select_experts(h, _t(logits, dev, torch.bfloat16), topk=k, renormalize=renorm, scoring_fn=scoring,
                            layer=layer, input_ids=_t(inp, dev))
    w_ref, ids_ref = routing.hash_select(logits, table, inp, renorm, scoring, 2.0)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.float().cpu().numpy(), w_ref, rtol=8e-3, atol=1e-6)
    if E == 4:
        assert ids.cpu().tolist() == [[2, 3], [0, 1]]
        np.testing.assert_array_equal(w.float().cpu().numpy(), np.full((2, 2), 0.5, np.float32))
