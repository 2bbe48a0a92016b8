"""GPU parity: row quantizer (bit-exact codes) and the grouped GEMM kinds
(skinny and tiled paths) against the CPU oracle."""

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
@pytest.mark.parametrize("block", [None, 128])
@pytest.mark.parametrize("M,K", [(1, 4096), (7, 2048), (64, 7168), (300, 1024),
                                 # decode rows on 1024 threads: held in registers, and streamed
                                 (3, 14336), (2, 40960),
                                 # prefill rows: held in registers up to 16384 columns, streamed beyond
                                 (4096, 4096), (600, 7168), (1000, 14336), (257, 16384), (300, 20480)])
def test_row_quant_runtime_bit_exact(dev, qdtype, block, M, K):
    if qdtype == "int8" and block is not None:
        pytest.skip("int8 activations are quantized per token only")
    from qmoe import ops

    print(f"row_quant {qdtype} block={block} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + K)
    x = _bf16(rng, (M, K), 3.0)
    x[0, :] = 0.0  # zero row -> scale 1
    if M > 2:
        x[2, 5] = 1e4  # large outlier
    x = codecs.bf16_round(x)  # the device sees bf16 values
    q_ref, s_ref = quant.quantize_act(x, qdtype, block=block)
    q, s = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype, block=block)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("M,K", [(600, 7168), (513, 14336)])
def test_row_quant_prefill_rows_non_finite(dev, qdtype, M, K):
    """Prefill rows with inf / NaN entries (and a row of zeros): the finite
    rows' codes and scales bit-exact against the oracle, the others' scales
    not finite (a row's inf or NaN does not leak into its neighbours)."""
    from qmoe import ops

    print(f"row_quant prefill rows non-finite {qdtype} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K)
    x = _bf16(rng, (M, K), 2.0)
    x[0, :] = 0.0
    x[3, 17] = np.inf
    x[5, K - 1] = -np.inf
    x[7, 4000] = np.nan
    x[M - 1, 9] = np.nan
    x[M - 1, K - 9] = -np.inf
    x = codecs.bf16_round(x)
    fin = np.isfinite(x).all(axis=1)
    assert fin.sum() == M - 4
    q_ref, s_ref = quant.quantize_act(x[fin], qdtype)
    q, s = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    sc = s.cpu().numpy()
    np.testing.assert_array_equal(sc[fin], s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy()[fin], q_ref.view(np.uint8))
    assert not np.isfinite(sc[~fin]).any()


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_row_quant_load_time_bit_exact(dev, qdtype):
    from qmoe import ops

    print(f"row_quant load {qdtype}", flush=True)
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((96, 1024)) * 0.02).astype(np.float32)
    w[5] = 0.0
    q_ref, s_ref = quant.quantize_tensor(w, qdtype)
    q, s = ops.row_quant(_t(w, dev), qdtype, mode="load")
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    assert s_ref[5] == 0.0


def test_e4m3_device_encoder_sweep(dev):
    """Every e4m3 rounding boundary (+-1 ulp) through the device encoder."""
    from qmoe import ops

    vals = codecs.e4m3_decode(np.arange(256, dtype=np.uint8))
    fin = np.unique(vals[np.isfinite(vals)].astype(np.float64))
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)
    x = np.concatenate([fin.astype(np.float32), mids, np.nextafter(mids, np.float32(1e9)),
                        np.nextafter(mids, np.float32(-1e9))]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    n = (x.size + 127) // 128 * 128
    row = np.zeros(n, np.float32)
    row[: x.size] = x
    row[-1] = 448.0  # absmax 448 -> load-time scale = 448 * f32(1/448) ~ 1
    xm = row.reshape(1, -1)
    q_ref, s_ref = quant.quantize_tensor(xm, "fp8")
    q, s = ops.row_quant(_t(xm, dev), "fp8", mode="load")
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def _bf16_neighbours(v):
    """bf16 values one bf16 ulp above and below each f32 value of v."""
    b = v.astype(np.float32).view(np.uint32) & 0xFFFF0000
    up = (b + 0x10000).view(np.float32)
    dn = (b - 0x10000).view(np.float32)
    return np.concatenate([up, dn])


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_runtime_encoder_sweep(dev, qdtype):
    """Runtime activation codes at every e4m3 rounding boundary (exact ties
    and one bf16 ulp either side), signed zeros and f32-subnormal-scale
    values, with the row scale exactly 1 (absmax 448 / 127) and 3."""
    from qmoe import ops

    qmax = 448.0 if qdtype == "fp8" else 127.0
    vals = codecs.e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    fin = np.unique(vals[np.isfinite(vals)])
    mids = (fin[:-1] + fin[1:]) / 2
    ints = np.arange(-128, 129, dtype=np.float64)
    halves = ints[:-1] + 0.5
    base = np.concatenate([fin, mids, ints, halves]).astype(np.float32)
    base = np.concatenate([base, _bf16_neighbours(base),
                           np.array([0.0, -0.0, 2.0 ** -10, -(2.0 ** -10), 3 * 2.0 ** -11, 2.0 ** -20,
                                     2.0 ** -126, -(2.0 ** -133)], np.float32)])
    rows = []
    for sc in (1.0, 3.0):
        x = codecs.bf16_round(base * np.float32(sc))
        x = x[np.abs(x) <= qmax * sc]
        n = (x.size + 127) // 128 * 128
        row = np.zeros(n, np.float32)
        row[: x.size] = x
        row[-1] = qmax * sc  # absmax -> scale exactly sc
        rows.append(row)
    n = max(r.size for r in rows)
    xm = np.zeros((len(rows), n), np.float32)
    for i, r in enumerate(rows):
        xm[i, : r.size] = r
        xm[i, -1] = r[-1]
    q_ref, s_ref = quant.quantize_act(xm, qdtype)
    q, s = ops.row_quant(_t(xm, dev, torch.bfloat16), qdtype)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))


@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_runtime_quant_division_stress(dev, qdtype):
    """Many quotients x / scale with scales that are not powers of two,
    against the oracle's IEEE division (codes and scales bit-exact)."""
    from qmoe import ops

    rng = np.random.default_rng(5)
    M, K = 48, 8192
    x = codecs.bf16_round((rng.uniform(-1, 1, (M, K)) * rng.uniform(0.01, 1000, (M, 1))).astype(np.float32))
    q_ref, s_ref = quant.quantize_act(x, qdtype)
    q, s = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref.view(np.uint8))
    if qdtype == "fp8":
        qb_ref, sb_ref = quant.quantize_act(x, qdtype, block=128)
        qb, sb = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype, block=128)
        np.testing.assert_array_equal(sb.cpu().numpy(), sb_ref)
        np.testing.assert_array_equal(qb.view(torch.uint8).cpu().numpy(), qb_ref.view(np.uint8))


# ------------------------------------------------------------------ GEMM

SHAPES_SKINNY = [(1, 512, 384), (8, 1024, 640), (16, 2048, 256), (33, 512, 4096), (64, 4096, 1024)]
# the last two split K across workgroups (few tiles, long K)
SHAPES_TILED = [(65, 512, 384), (200, 1024, 1000), (512, 2048, 2048), (300, 1536, 2304), (130, 8192, 512),
                (96, 14336, 768), (200, 8192, 640)]


@pytest.mark.parametrize("M,K,N", SHAPES_SKINNY + SHAPES_TILED)
def test_w8a8_fp8_per_channel(dev, M, K, N):
    from qmoe import _capi, ops

    print(f"w8a8 fp8 pc M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + K + N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = _bf16(rng, (M, K))
    ref, xq_ref, xs_ref = linear.w8a8_per_channel(x, wq, ws, "fp8")
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), xq_ref)
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq, dev), a_scale=xs, w_scale=_t(ws, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"fp8 pc {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", SHAPES_SKINNY + SHAPES_TILED)
def test_w8a8_int8_per_channel_bit_exact(dev, M, K, N):
    """int32 accumulation is exact, so the f32 epilogue in the reference's
    operation order reproduces the oracle bit for bit."""
    from qmoe import _capi, ops

    print(f"w8a8 int8 pc M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M * 3 + K + N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "int8")
    x = _bf16(rng, (M, K))
    ref, xq_ref, _ = linear.w8a8_per_channel(x, wq, ws, "int8")
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "int8")
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq.view(np.uint8), dev), a_scale=xs,
                 w_scale=_t(ws, dev), wfmt=1)
    np.testing.assert_array_equal(y.float().cpu().numpy(), ref)


# 128-row weight tiles (dense per-channel problems whose 256-row tiles leave
# CUs idle): ragged token and channel tiles, the tall-K forms with and
# without a K split
SHAPES_NARROW = [(64, 4096, 14336), (100, 4096, 2048), (256, 2048, 1000), (300, 14336, 1024), (700, 8192, 1152),
                 # at most 1024 channels, over 256 tokens: 64- and 128-token tiles
                 (2000, 7168, 576), (4096, 4096, 1000)]


@pytest.mark.parametrize("M,K,N", SHAPES_NARROW)
@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_w8a8_narrow_weight_tiles(dev, M, K, N, qdtype):
    """The 1-byte tile kernel with 128-row weight tiles against the oracle
    (FP8 within one bf16 ulp of the same-code oracle, INT8 bit-exact), with
    a bias on the FP8 runs; the plan reports the narrow tiles."""
    from qmoe import _capi, ops

    wf = int(qdtype == "int8")
    plan = ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)
    print(f"w8a8 narrow {qdtype} M={M} K={K} N={N} plan={plan}", flush=True)
    assert plan[4] == "tiled_1b_n128", plan
    rng = np.random.default_rng(M + 3 * K + N + wf)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    x = _bf16(rng, (M, K))
    bias = None if wf else codecs.bf16_round(rng.standard_normal(N).astype(np.float32))
    ref, _, _ = linear.w8a8_per_channel(x, wq, ws, qdtype)
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq.view(np.uint8), dev), a_scale=xs,
                 w_scale=_t(ws, dev), wfmt=wf, bias=None if bias is None else _t(bias, dev))
    got = y.float().cpu().numpy()
    if wf:
        np.testing.assert_array_equal(got, ref)
    else:
        # the bias is added to the f32 result before the bf16 rounding
        xq_r, xs_r = quant.quantize_act(x, "fp8")
        dot = np.matmul(codecs.e4m3_decode(xq_r), codecs.e4m3_decode(wq).T).astype(np.float32)
        full = ((dot * xs_r[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32) + bias[None, :]
        assert_close_same_codes(got, codecs.bf16_round(full.astype(np.float32)), f"narrow fp8 {M}x{K}x{N}")


# more 256 x 256 tiles than CUs: persistent workgroups (ragged last token
# and channel tiles, the shortest K of the path, a tile count that leaves
# workgroups with different numbers of tiles)
SHAPES_PERSISTENT = [(2000, 1024, 8200), (4096, 512, 4352), (1300, 2048, 14336)]


@pytest.mark.parametrize("M,K,N", SHAPES_PERSISTENT)
@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
@pytest.mark.parametrize("pbn", ["256", "224"])
def test_w8a8_persistent_tiles(dev, monkeypatch, M, K, N, qdtype, pbn):
    """The persistent kernel in both tile heights (256 x 256, and 256
    tokens x 224 weight rows: ragged channel tiles at N 8200 and 4352)
    against the oracle (FP8 within one bf16 ulp of the same-code oracle, INT8
    bit-exact), and the plan reports it."""
    from qmoe import _capi, ops

    monkeypatch.setenv("QMOE_F8_PERSIST_BN", pbn)
    wf = int(qdtype == "int8")
    plan = ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)
    print(f"w8a8 persistent {qdtype} M={M} K={K} N={N} rows={pbn} plan={plan}", flush=True)
    assert plan[4:] == ("tiled_1b_persistent", 256, 1), plan
    rng = np.random.default_rng(M + 5 * K + N + wf)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    x = _bf16(rng, (M, K))
    ref, xq_ref, _ = linear.w8a8_per_channel(x, wq, ws, qdtype)
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), xq_ref.view(np.uint8))
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq.view(np.uint8), dev), a_scale=xs,
                 w_scale=_t(ws, dev), wfmt=wf)
    got = y.float().cpu().numpy()
    if qdtype == "int8":
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_same_codes(got, ref, f"fp8 persistent {M}x{K}x{N}")


# output rows of a multiple of 32 KB with short K: the persistent tiles in
# plain order (the in-flight stores then spread over the whole row width)
@pytest.mark.parametrize("M,K,N", [(1024, 512, 16384), (600, 1024, 32768),
                                   # 128 x 224 tiles (mid-size problem)
                                   (300, 1024, 16384)])
@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_w8a8_persistent_wide_rows(dev, monkeypatch, M, K, N, qdtype):
    """Plain tile order against the oracle (sampled rows: FP8 within one bf16
    ulp of the same-code oracle, INT8 bit-exact) and bit-identical to the
    XCD-run order (QMOE_F8_PERSIST_ORDER=0)."""
    from qmoe import _capi, ops

    wf = int(qdtype == "int8")
    rng = np.random.default_rng(M + K + N + wf)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    x = _bf16(rng, (M, K))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    wt, wst = _t(wq.view(np.uint8), dev), _t(ws, dev)
    with ops.record_plans() as plans:
        y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=wf)
    print(f"w8a8 persistent wide rows {qdtype} M={M} K={K} N={N} plan={plans[0]}", flush=True)
    assert plans[0][4] == "tiled_1b_persistent", plans
    monkeypatch.setenv("QMOE_F8_PERSIST_ORDER", "0")
    y0 = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=wf)
    assert torch.equal(y.view(torch.int16), y0.view(torch.int16))
    r = np.unique(np.linspace(0, M - 1, 6).round().astype(np.int64))
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, qdtype)
    got = y[torch.from_numpy(r).to(dev)].float().cpu().numpy()
    if wf:
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_same_codes(got, ref, f"persistent wide rows {M}x{K}x{N}")


@pytest.mark.parametrize("seed", range(4))
def test_w8a8_persistent_matches_one_tile(dev, monkeypatch, seed):
    """Seeded shapes of 300-5000 tokens, 1000-20000 output channels (N % 8 ==
    0) and K of 512-4096: whatever persistent tile shape the planner picks
    (256 x 256, 256 x 224, 128 x 224), the outputs equal the one-tile
    kernel's bit for bit (both run the same MFMA sequence per output)."""
    from qmoe import _capi, ops

    rng = np.random.default_rng(1000 + seed)
    for _ in range(4):
        M = int(rng.integers(300, 5000))
        N = int(rng.integers(125, 2500)) * 8
        K = int(rng.integers(2, 17)) * 256
        wf = int(rng.integers(0, 2))
        monkeypatch.delenv("QMOE_F8_PERSIST", raising=False)
        plan = ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)
        print(f"w8a8 persistent vs one-tile M={M} K={K} N={N} wfmt={wf} plan={plan}", flush=True)
        g = torch.Generator(device=dev).manual_seed(seed * 7 + M)
        q = torch.randint(0, 120, (N, K), device=dev, dtype=torch.uint8, generator=g)
        if wf:
            q = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g).view(torch.uint8)
        xq = torch.randint(0, 120, (M, K), device=dev, dtype=torch.uint8, generator=g)
        if wf:
            xq = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g).view(torch.uint8)
        s = torch.rand(N, device=dev, generator=g) * 1e-3
        xs = torch.rand(M, device=dev, generator=g)
        y = ops.gemm(_capi.W8A8_PC, xq, q, a_scale=xs, w_scale=s, wfmt=wf)
        monkeypatch.setenv("QMOE_F8_PERSIST", "0")
        assert ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)[4] != "tiled_1b_persistent"
        y1 = ops.gemm(_capi.W8A8_PC, xq, q, a_scale=xs, w_scale=s, wfmt=wf)
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16)), (M, K, N, wf, plan)


@pytest.mark.parametrize("M,K,N", [(1000, 2048, 7000), (512, 4096, 14336), (300, 1024, 14336)])
@pytest.mark.parametrize("qdtype", ["fp8", "int8"])
def test_w8a8_persistent_mid_tiles(dev, monkeypatch, M, K, N, qdtype):
    """Mid-size problems whose 64- or 128-token one-tile grid takes more
    tile rounds x area run the persistent kernel in 128-token x 224-row tiles
    (ragged last token and channel tiles at 1000 x 7000 and 300 tokens; 300
    tokens would take 64-token one-tile tiles): against the oracle, and
    bit-identical to the one-tile kernel (the same MFMA sequence per
    output)."""
    from qmoe import _capi, ops

    wf = int(qdtype == "int8")
    plan = ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)
    print(f"w8a8 persistent mid {qdtype} M={M} K={K} N={N} plan={plan}", flush=True)
    assert plan[4:] == ("tiled_1b_persistent", 128, 1), plan
    rng = np.random.default_rng(M + 3 * K + N + wf)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, qdtype)
    x = _bf16(rng, (M, K))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), qdtype)
    wt, wst = _t(wq.view(np.uint8), dev), _t(ws, dev)
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=wf)
    monkeypatch.setenv("QMOE_F8_PERSIST_BN", "256")  # the one-tile 128 x 256 kernel
    y1 = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst, wfmt=wf)
    assert ops.plan_for_shape(_capi.W8A8_PC, M, N, K, wfmt=wf)[4] == "tiled_1b"
    assert torch.equal(y.view(torch.int16), y1.view(torch.int16))
    r = np.unique(np.linspace(0, M - 1, 6).round().astype(np.int64))
    ref, _, _ = linear.w8a8_per_channel(x[r], wq, ws, qdtype)
    got = y[torch.from_numpy(r).to(dev)].float().cpu().numpy()
    if qdtype == "int8":
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close_same_codes(got, ref, f"fp8 persistent mid {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (32, 2048, 768), (130, 1024, 640), (256, 2048, 1024),
                                   # tiled block-scaled kernel: ragged tiles, 32/64/128-token tiles,
                                   # a K split (tall K, few tokens)
                                   (300, 2048, 1280), (70, 1536, 384), (400, 1024, 2304), (96, 8192, 512),
                                   # wide N (>= 16384 channels): tiled from 17 rows, K split 2 up to
                                   # 32 tokens, 128-row weight tiles from 33 to 128 and from 257 to
                                   # 512 tokens (tile scales)
                                   (17, 1024, 16384), (50, 768, 16384), (100, 512, 16512), (260, 512, 16384)])
@pytest.mark.parametrize("tile_scales", [True, False])
def test_w8a8_fp8_block(dev, M, K, N, tile_scales):
    from qmoe import _capi, ops

    print(f"w8a8 blk M={M} K={K} N={N} tiles={tile_scales}", flush=True)
    rng = np.random.default_rng(M + 2 * K + N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if tile_scales:
        wq, st = quant.quantize_fp8_tiles(w)
        sblk, bn, s_dev = linear.tile_scales_to_blocks(st, N), 128, st
    else:
        wq, sblk = quant.quantize_tensor(w, "fp8", block=128)
        bn, s_dev = 1, sblk
    x = _bf16(rng, (M, K))
    ref, xq_ref, _ = linear.w8a8_blockwise(x, wq, sblk)
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8", block=128)
    np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), xq_ref)
    y = ops.gemm(_capi.W8A8_BLK, xq.view(torch.uint8), _t(wq, dev), a_scale=xs,
                 w_scale=_t(s_dev, dev), ws_bn=bn)
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"fp8 blk {M}x{K}x{N}")


def _nv_scales(rng, n, k):
    """Fused NVFP4 block scales as a checkpoint makes them: e4m3 block scale
    times a float32 global with a full mantissa (so the bf16 rounding of the
    product matters), [n, k/16] float32."""
    blk = codecs.e4m3_decode(rng.integers(0x20, 0x48, (n, k // 16)).astype(np.uint8))
    return codecs.nvfp4_fuse_scales(blk, np.float32(0.0123456789))


@pytest.mark.parametrize("M,K,N", [(1, 2880, 5760), (16, 2880, 5760), (5, 512, 200), (33, 1024, 96),
                                   # K % 128 != 0 (streaming kernel's tail step), small K
                                   (3, 2848, 200), (1, 416, 70), (7, 96, 130),
                                   # tiled kernel: 64/128-token tiles, K splits, ragged tiles
                                   (300, 2880, 768), (520, 1024, 512), (200, 4096, 4096), (50, 2880, 1000),
                                   # K % 64 == 32 above the streaming bound: 64-row streaming passes
                                   (70, 2848, 300)])
def test_w4a16_nvfp4(dev, M, K, N):
    from qmoe import _capi, ops

    print(f"w4a16 nv M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + 2 * K + N)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = _nv_scales(rng, N, K)
    x = _bf16(rng, (M, K))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref = linear.w4a16_nvfp4(x, packed, sc, bias)
    y = ops.gemm(_capi.W4A16_NV, _t(x, dev, torch.bfloat16), _t(packed, dev),
                 w_scale=_t(sc, dev, torch.bfloat16), bias=_t(bias, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"nvfp4 {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(16, 2880, 320), (256, 4096, 512)])
def test_w4a16_nvfp4_dequant_bit_exact(dev, M, K, N):
    """One-hot activation rows read single dequantized weights back: output
    row i is column k_i of bf16(code * bf16(scale)), exactly (one nonzero
    product, f32 accumulation, a bf16 value rounded to bf16). M = 16 runs the
    streaming kernel, M = 256 the tiled one; the k_i cover every 16-k block
    position of a row."""
    from qmoe import _capi, ops

    print(f"w4a16 nv one-hot M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(K + N)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = _nv_scales(rng, N, K)
    ks = (np.arange(M) * (K // M) + np.arange(M) % 16) % K
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    y = ops.gemm(_capi.W4A16_NV, _t(x, dev, torch.bfloat16), _t(packed, dev), w_scale=_t(sc, dev, torch.bfloat16))
    want = codecs.dequant_nvfp4(packed, sc)[:, ks].T
    np.testing.assert_array_equal(y.float().cpu().numpy(), want)


def _int4_case(rng, n, k, group):
    """Packed-int4 weights (int32 carriers, compressed-tensors encoding) and
    bf16-valued group scales."""
    carriers = codecs.int4_pack(rng.integers(-8, 8, (n, k)))
    sc = codecs.bf16_round((rng.random((n, k // group)) * 0.02 + 0.002).astype(np.float32))
    return carriers, sc


@pytest.mark.parametrize("M,K,N,group", [(1, 2880, 5760, 32), (16, 4096, 1024, 128), (5, 512, 200, 64),
                                         # K % 128 != 0: the streaming kernel's tail step
                                         (3, 2848, 200, 32), (7, 96, 130, 32), (2, 320, 64, 64),
                                         # tiled kernel (groups straddle and fill 64-k stages)
                                         (300, 2880, 768, 32), (520, 1024, 512, 128), (200, 4096, 1024, 64),
                                         (256, 2880, 1000, 32), (400, 2048, 768, 64),
                                         # K % 64 == 32 above the streaming bound: 64-row streaming passes
                                         (70, 2848, 300, 32)])
def test_w4a16_int4(dev, M, K, N, group):
    from qmoe import _capi, ops

    print(f"w4a16 int4 M={M} K={K} N={N} group={group}", flush=True)
    rng = np.random.default_rng(M + K + N + group)
    carriers, sc = _int4_case(rng, N, K, group)
    x = _bf16(rng, (M, K))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref = linear.w4a16_int4(x, carriers, sc, bias)
    y = ops.gemm(_capi.W4A16_I4, _t(x, dev, torch.bfloat16), _t(carriers, dev).view(torch.uint8),
                 w_scale=_t(sc, dev, torch.bfloat16), bias=_t(bias, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"int4 {M}x{K}x{N} g{group}")


@pytest.mark.parametrize("M,K,N,group", [(16, 2048, 320, 32), (16, 4096, 256, 128), (256, 4096, 512, 64),
                                         (256, 2048, 256, 128)])
def test_w4a16_int4_dequant_bit_exact(dev, M, K, N, group):
    """One-hot activation rows read single dequantized weights back (as for
    NVFP4): bf16(value * scale) exactly, through the streaming (M = 16) and
    the tiled (M = 256) kernel."""
    from qmoe import _capi, ops

    print(f"w4a16 int4 one-hot M={M} K={K} N={N} group={group}", flush=True)
    rng = np.random.default_rng(K + N + group)
    carriers, sc = _int4_case(rng, N, K, group)
    sc = codecs.bf16_round(sc * np.float32(1.0 + 3.0 / 512))  # mantissas that make products round
    ks = (np.arange(M) * (K // M) + np.arange(M) * 7) % K
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    y = ops.gemm(_capi.W4A16_I4, _t(x, dev, torch.bfloat16), _t(carriers, dev).view(torch.uint8),
                 w_scale=_t(sc, dev, torch.bfloat16))
    want = codecs.dequant_int4(carriers, sc)[:, ks].T
    np.testing.assert_array_equal(y.float().cpu().numpy(), want)


@pytest.mark.parametrize("M,K,N", [(1, 2880, 5760), (16, 2880, 5760), (128, 2880, 1440),
                                   (5, 512, 200), (90, 1024, 96),
                                   # K % 256 = 32, 160 and K < 256: every partial last step pair
                                   (3, 2848, 200), (1, 416, 70), (7, 96, 130), (2, 160, 64),
                                   # e8m0 rows longer than one staging batch of the streaming kernel
                                   (1, 8192, 256), (2, 16384, 64),
                                   # tiled kernel: 32/64/128-token tiles, K splits, ragged tiles;
                                   # K % 64 != 0 takes the generic tiled kernel
                                   (300, 2880, 768), (520, 1024, 512), (600, 512, 9216), (1200, 512, 9216),
                                   (70, 2848, 300),
                                   # 33..64 rows: the streaming kernel in 16-row slices
                                   (50, 2880, 1000)])
def test_w4a16_mxfp4(dev, M, K, N):
    from qmoe import _capi, ops

    print(f"w4a16 mx M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + K + 3 * N)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = (127 + rng.integers(-8, 1, (N, K // 32))).astype(np.uint8)
    x = _bf16(rng, (M, K))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    ref = linear.w4a16_mxfp4(x, packed, sc, bias)
    y = ops.gemm(_capi.W4A16_MX, _t(x, dev, torch.bfloat16), _t(packed, dev), w_scale=_t(sc, dev),
                 bias=_t(bias, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, f"mxfp4 {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (48, 512, 384), (100, 1024, 512)])
def test_w8a16_and_w16a16(dev, M, K, N):
    from qmoe import _capi, ops

    print(f"w8a16/w16a16 M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + K + 5 * N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = _bf16(rng, (M, K))
    xt = _t(x, dev, torch.bfloat16)
    ref = linear.w8a16_per_channel(x, wq, ws)
    y = ops.gemm(_capi.W8A16_PC, xt, _t(wq, dev), w_scale=_t(ws, dev))
    assert_close_same_codes(y.float().cpu().numpy(), ref, "w8a16")
    wb = codecs.bf16_round(w)
    ref = linear.w16a16(x, wb)
    y = ops.gemm(_capi.W16A16, xt, _t(wb, dev, torch.bfloat16))
    assert_close_same_codes(y.float().cpu().numpy(), ref, "w16a16")


@pytest.mark.parametrize("kind", ["w16a16", "w8a16_pc", "w8a16_blk"])
@pytest.mark.parametrize("M,K,N,ks", [(4096, 7168, 256, 8), (8192, 7168, 256, 4), (300, 4096, 512, 8),
                                      (1000, 2048, 384, 4), (2000, 4096, 200, 8), (129, 7168, 256, 8)])
def test_tiled_generic_k_split(dev, monkeypatch, kind, M, K, N, ks):
    """The generic tiled kernel split over K (dense bf16 activations in
    under 256 tiles of 128 x 128; each slice's f32 sums summed in
    slice order by the finishing kernel, which applies the weight scale, bias
    and row weight): the planned split, oracle rows to the same-codes bar, and
    the unsplit kernel (QMOE_TILED_KSPLIT=1) with bias and row weights."""
    from qmoe import _capi, ops

    print(f"tiled generic K split {kind} M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = _bf16(rng, (M, K))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    r = np.unique(np.linspace(0, M - 1, 6).round().astype(np.int64))
    if kind == "w16a16":
        wb = codecs.bf16_round(w)
        kc, wt, kw = _capi.W16A16, _t(wb, dev, torch.bfloat16), {}
        ref = linear.w16a16(x[r], wb, bias=bias)
    elif kind == "w8a16_pc":
        wq, ws = quant.quantize_tensor(w, "fp8")
        kc, wt, kw = _capi.W8A16_PC, _t(wq, dev), dict(w_scale=_t(ws, dev))
        ref = linear.w8a16_per_channel(x[r], wq, ws)  # no bias term in this oracle
    else:
        wq, sblk = quant.quantize_tensor(w, "fp8", block=128)
        kc, wt, kw = _capi.W8A16_BLK, _t(wq, dev), dict(w_scale=_t(sblk, dev), ws_bn=1)
        ref = linear.w8a16_blockwise(x[r], wq, sblk, bias=bias)
    xt, bt = _t(x, dev, torch.bfloat16), _t(bias, dev)
    with ops.record_plans() as plans:
        y = ops.gemm(kc, xt, wt, bias=None if kind == "w8a16_pc" else bt, **kw)
    assert plans[0][4:] == ("tiled_generic", 128, ks), plans
    assert_close_same_codes(y[torch.from_numpy(r).to(dev)].float().cpu().numpy(), ref, f"{kind} split M={M}")
    rw = _t(rng.uniform(0.25, 2.0, M).astype(np.float32), dev, torch.bfloat16)
    y2 = ops.gemm(kc, xt, wt, bias=bt, row_weight=rw, **kw)
    monkeypatch.setenv("QMOE_TILED_KSPLIT", "1")
    with ops.record_plans() as plans:
        y1 = ops.gemm(kc, xt, wt, bias=bt, row_weight=rw, **kw)
    assert plans[0][4:] == ("tiled_generic", 128, 1), plans
    assert_close_same_codes(y2.float().cpu().numpy(), y1.float().cpu().numpy(), f"{kind} split vs one pass M={M}")


def test_split_k_deterministic_and_reusable(dev):
    """Split-K (slices summed in a fixed order by a second kernel) gives
    identical results on repeat calls that share the workspace."""
    from qmoe import _capi, ops

    rng = np.random.default_rng(21)
    K, N = 14336, 1024
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = _bf16(rng, (4, K))
    ref, _, _ = linear.w8a8_per_channel(x, wq, ws, "fp8")
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    wt, wst = _t(wq, dev), _t(ws, dev)
    outs = [ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), wt, a_scale=xs, w_scale=wst) for _ in range(3)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert_close_same_codes(outs[0].float().cpu().numpy(), ref, "split-k")


@pytest.mark.parametrize("M,K,I", [(200, 1024, 384), (96, 8192, 256)])
def test_w8a8_fp8_block_fused_activation(dev, M, K, I):
    """Block-scaled FP8 GEMM with the gate/up SwiGLU fused (DeepSeek shared
    expert form), with and without a K split."""
    from qmoe import _capi, ops

    print(f"w8a8 blk act M={M} K={K} I={I}", flush=True)
    rng = np.random.default_rng(M + K + I)
    w = (rng.standard_normal((2 * I, K)) * 0.02).astype(np.float32)
    wq, st = quant.quantize_fp8_tiles(w)
    x = _bf16(rng, (M, K))
    gu, _, _ = linear.w8a8_blockwise(x, wq, linear.tile_scales_to_blocks(st, 2 * I), round_out=False)
    ref = codecs.bf16_round(omoe.act_fn(gu[:, :I].astype(np.float32), gu[:, I:].astype(np.float32), "silu"))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8", block=128)
    y = ops.gemm(_capi.W8A8_BLK, xq.view(torch.uint8), _t(wq, dev), a_scale=xs, w_scale=_t(st, dev),
                 ws_bn=128, activation="silu")
    assert_close_rows(y.float().cpu().numpy(), ref, f"fp8 blk silu {M}x{K}x{I}")


@pytest.mark.parametrize("act", ["silu", "swigluoai", "gelu", "gelu_tanh", "silu_and_mul_with_clamp",
                                 "situ:2.0:none", "situ:1.5:3.0"])
def test_tiled_split_k_fused_activation(dev, act):
    """Tiled FP8 GEMM with a K split and the gate/up activation applied by
    the split-K finishing kernel."""
    from qmoe import _capi, ops

    print(f"tiled split-k act {act}", flush=True)
    rng = np.random.default_rng(5)
    M, K, I = 100, 8192, 320
    w = (rng.standard_normal((2 * I, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = _bf16(rng, (M, K))
    xq_ref, sx = quant.quantize_act(x, "fp8")
    acc = codecs.e4m3_decode(xq_ref).astype(np.float64) @ codecs.e4m3_decode(wq).astype(np.float64).T
    gu = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
    ref = codecs.bf16_round(omoe.act_fn(gu[:, :I], gu[:, I:], act))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq, dev), a_scale=xs, w_scale=_t(ws, dev),
                 activation=act)
    assert_close_rows(y.float().cpu().numpy(), ref, f"split-k {act}")



ACTS = ["silu", "swigluoai", "gelu", "gelu_tanh", "silu_and_mul_with_clamp", "situ:2.0:none", "situ:1.5:3.0"]


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("M", [8, 200])
def test_fused_activation_strings(dev, act, M):
    """Every activation string of `kernels/megablox/gmm_v2.py:101-122` fused
    into the gate/up epilogue, through the streaming (M = 8) and the tiled
    (M = 200) kernels, FP8 per-channel weights. Gate/up sums are scaled
    up so that the clamps (7, 10) and the tanh saturations are reached."""
    from qmoe import _capi, ops

    print(f"fused act {act} M={M}", flush=True)
    rng = np.random.default_rng(M + len(act))
    K, I = 1024, 384
    w = (rng.standard_normal((2 * I, K)) * 0.4).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = _bf16(rng, (M, K))
    xq_ref, sx = quant.quantize_act(x, "fp8")
    acc = codecs.e4m3_decode(xq_ref).astype(np.float64) @ codecs.e4m3_decode(wq).astype(np.float64).T
    gu = ((acc.astype(np.float32) * sx[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
    assert np.abs(gu).max() > 12.0  # the clamps bind
    ref = codecs.bf16_round(omoe.act_fn(gu[:, :I], gu[:, I:], act))
    xq, xs = ops.row_quant(_t(x, dev, torch.bfloat16), "fp8")
    y = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), _t(wq, dev), a_scale=xs, w_scale=_t(ws, dev),
                 activation=act)
    assert_close_rows(y.float().cpu().numpy(), ref, f"act {act} M={M}")


# e8m0 bytes with known answers in the reference's decoder tests
# (`tests/layers/core/test_mxfp4_requantization.py:194-209`)
E8M0_EDGE = [0, 1, 127, 128, 253, 254, 255]


@pytest.mark.parametrize("M", [16, 256])
def test_mxfp4_one_hot_dequant_e8m0_edges(dev, M):
    """One-hot activation rows read single dequantized MXFP4 weights back
    through the streaming (M = 16) and tiled (M = 256) kernels, with the e8m0
    edge bytes 0 (2^-127, an f32 subnormal), 1, 127, 128, 253, 254 and 255
    (+inf) among the block scales. Rows holding only finite weights must read
    back LUT[code] * 2^(byte - 127) exactly (bf16 values; subnormals kept);
    the oracle's own matmul defines the rows that hold an inf (0 * inf = NaN
    there)."""
    from qmoe import _capi, ops

    print(f"mxfp4 one-hot e8m0 edges M={M}", flush=True)
    K, N = 1024, 256
    rng = np.random.default_rng(M)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = np.full((N, K // 32), 127, np.uint8)
    safe = np.array([0, 1, 127, 128], np.uint8)
    # rows 0..N/2: every block scale from {0, 1, 127, 128} (finite weights)
    sc[: N // 2] = safe[rng.integers(0, 4, (N // 2, K // 32))]
    # rows N/2..: the large bytes too (weights up to 6 * 2^127: inf in f32)
    sc[N // 2:] = np.array(E8M0_EDGE, np.uint8)[rng.integers(0, 7, (N - N // 2, K // 32))]
    ks = (np.arange(M) * (K // M) + np.arange(M) * 5) % K
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    y = ops.gemm(_capi.W4A16_MX, _t(x, dev, torch.bfloat16), _t(packed, dev), w_scale=_t(sc, dev))
    got = y.float().cpu().numpy()
    deq = codecs.dequant_mxfp4(packed, sc)
    want = deq[:, ks].T  # [M, N]
    fin = np.isfinite(deq).all(axis=1)  # rows whose every weight is finite
    assert fin[: N // 2].all() and not fin.all()
    np.testing.assert_array_equal(got[:, fin], want[:, fin])
    sub = (sc[: N // 2] == 0).any()
    assert sub, "subnormal scales are exercised"
    with np.errstate(invalid="ignore", over="ignore"):
        ref = linear.w4a16_mxfp4(x, packed, sc)
    np.testing.assert_array_equal(np.isnan(got[:, ~fin]), np.isnan(ref[:, ~fin]))
