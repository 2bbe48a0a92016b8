"""Pins of the fused decode MoE oracle (`oracle/decode.py`, CPU).

* the quantizer: hand-worked float32 values (scale max/448, reciprocal
  multiply, e4m3 round to nearest even), partial and zero blocks;
* the reference's own test (`tests/kernels/experimental/
  test_fused_moe_decode_kernel.py:87-143, 280-311`): the layer within 0.08
  (max over rows of the relative row-norm error) of the decomposed float
  layer, with its positive controls -- dropping one routed expert, or
  scaling the shared expert by routed_scale, must exceed 0.08 -- for the
  gated (Qwen3.5) and the ungated + routed_scale 2.5 (GLM) conventions;
* exact identities: a power-of-two route weight scales the routed term
  exactly (the coefficient multiplies before the second quantization, which
  is scale-invariant); the shared expert is the same computation as a routed
  expert of weight 1; duplicate route ids sum their bf16 weights.
"""

import numpy as np
import pytest

from oracle import codecs, decode, quant


def _bf(v):
    return codecs.bf16_round(np.asarray(v, np.float32))


def test_quantizer_known_answers():
    """absmax 448 -> scale 1 (codes exact); absmax 1 -> scale f32(1/448),
    inv = f32(1/scale) = 448.00003, 0.1 -> 44.8 -> e4m3 44 (0x63), 1 -> 448
    (0x7E); a zero block keeps scale 0 and codes 0; blocks start at column
    0 and the last one may be partial."""
    x = np.zeros((3, 640), np.float32)
    x[0, :5] = [448.0, 1.0, -0.5, 3.0, 0.0]
    x[1, :3] = [1.0, 0.1, -1.0]
    x[2, 520] = -2.0  # only the partial block
    q, s = decode.quantize_rows_f32(x, 512)
    assert s.shape == (3, 2)
    assert s[0, 0] == 1.0 and s[0, 1] == 0.0
    assert q[0, :5].tolist() == [0x7E, 0x38, 0xB0, 0x44, 0x00]
    assert s[1, 0] == np.float32(1.0) / np.float32(448.0)
    assert q[1, :3].tolist() == [0x7E, 0x63, 0xFE]
    assert s[2, 0] == 0.0 and (q[2, :512] == 0).all()
    assert s[2, 1] == np.float32(2.0) / np.float32(448.0) and q[2, 520] == 0xFE
    # the reciprocal-multiply recipe differs from the runtime quantizer's
    # division on some inputs, and agrees with it at power-of-two scales
    rng = np.random.default_rng(0)
    xr = _bf(rng.standard_normal((64, 512)).astype(np.float32))
    qd, _ = decode.quantize_rows_f32(xr, 512)
    qr, _ = quant.quantize_act(xr, "fp8", block=512)
    assert (qd != qr).any() and (qd == qr).mean() > 0.99
    xp = xr.copy()
    xp[:, 0] = 448.0 * 2.0 ** rng.integers(-4, 4, 64)
    xp[:, 1:] = np.clip(xp[:, 1:], -1.0, 1.0)
    np.testing.assert_array_equal(decode.quantize_rows_f32(xp, 512)[0], quant.quantize_act(xp, "fp8", block=512)[0])


def _q_rows(w):
    """Per-output-channel e4m3 quantization of N-major weights, the reference
    test's `q(w, axis)` (`test_fused_moe_decode_kernel.py:54-56`); the codes
    come from torch's cast (the oracle's encoder is pinned to it), which is
    much faster at these sizes."""
    import torch

    s = (np.abs(w).max(axis=-1, keepdims=True) / 448.0).astype(np.float32)
    q = torch.from_numpy(np.ascontiguousarray(w / s)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q, s[..., 0]


def _layer(seed, E=64, H=1024, I=256, Is=128, T=8, k=10, tiles=False):
    rng = np.random.default_rng(seed)
    if tiles:
        w1q, w1s = zip(*[quant.quantize_fp8_tiles((rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32))
                         for _ in range(E)])
        w2q, w2s = zip(*[quant.quantize_fp8_tiles((rng.standard_normal((H, I)) * 0.02).astype(np.float32))
                         for _ in range(E)])
        w1q, w1s, w2q, w2s = map(np.stack, (w1q, w1s, w2q, w2s))
        sw1q, sw1s = quant.quantize_fp8_tiles((rng.standard_normal((2 * Is, H)) * 0.02).astype(np.float32))
        sw2q, sw2s = quant.quantize_fp8_tiles((rng.standard_normal((H, Is)) * 0.02).astype(np.float32))
    else:
        w1q, w1s = _q_rows(rng.standard_normal((E, 2 * I, H), dtype=np.float32) * np.float32(0.02))
        w2q, w2s = _q_rows(rng.standard_normal((E, H, I), dtype=np.float32) * np.float32(0.02))
        sw1q, sw1s = _q_rows((rng.standard_normal((2 * Is, H)) * 0.02).astype(np.float32))
        sw2q, sw2s = _q_rows((rng.standard_normal((H, Is)) * 0.02).astype(np.float32))
    gate = _bf(rng.normal(size=H) * 0.02)
    x = _bf(rng.normal(size=(T, H)))
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    tw = _bf(rng.dirichlet(np.ones(k), size=T))
    return dict(hidden=x, w1q=w1q, w1s=w1s, w2q=w2q, w2s=w2s, shared_w1q=sw1q, shared_w1s=sw1s,
                shared_w2q=sw2q, shared_w2s=sw2s, shared_gate=gate, topk_weights=tw, topk_ids=ids,
                weight_blocks=128 if tiles else None)


def _heaviest(L):
    """Token 0's expert of largest route weight: the positive control drops
    it (the reference test drops ids[0, 0], whose weight may be small)."""
    return int(L["topk_ids"][0, np.argmax(L["topk_weights"][0])])


def _max_rel(a, ref):
    """The reference test's bar (`test_fused_moe_decode_kernel.py:270-277`)."""
    return (np.linalg.norm(a - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)).max()


@pytest.mark.parametrize("m,padded", [(8, False), (8, True), (32, False)])
def test_matches_decomposed_layer_gated(m, padded):
    L = _layer(seed=m, T=m)
    if padded:
        L["topk_weights"][m - 3:] = 0.0  # zero-weight tokens: shared expert only
    got = decode.fused_moe_decode(**L)
    ref = decode.decomposed_layer_f32(**L)
    assert np.isfinite(got).all()
    assert _max_rel(got, ref) < 0.08
    broken = decode.decomposed_layer_f32(**L, skip_expert=_heaviest(L))
    assert _max_rel(got, broken) > 0.08


def test_ungated_shared_expert_routed_scale():
    """GLM-5.2 convention: ungated shared expert, routed_scale 2.5 on the
    routed sum only (`test_fused_moe_decode_kernel.py:300-311`)."""
    L = _layer(seed=5, T=8)
    L["shared_gate"] = None
    got = decode.fused_moe_decode(**L, routed_scale=2.5)
    ref = decode.decomposed_layer_f32(**L, routed_scale=2.5)
    assert _max_rel(got, ref) < 0.08
    # scaling the shared expert too is wrong and fails the bar
    shared_only = decode.decomposed_layer_f32(**{**L, "topk_weights": np.zeros_like(L["topk_weights"])})
    wrong = ref + 1.5 * shared_only
    assert _max_rel(got, wrong) > 0.08


def test_tile_weights_match_decomposed_layer():
    """The 128x128-tile variant against the same decomposed layer (tile
    scales dequantized per 128x128 block)."""
    L = _layer(seed=7, E=16, H=1024, I=256, Is=256, T=4, k=4, tiles=True)
    got = decode.fused_moe_decode(**L)
    ref = decode.decomposed_layer_f32(**L)
    assert _max_rel(got, ref) < 0.08
    broken = decode.decomposed_layer_f32(**L, skip_expert=_heaviest(L))
    assert _max_rel(got, broken) > 0.08


@pytest.mark.parametrize("tiles", [False, True])
def test_power_of_two_route_weight_scales_the_routed_term_exactly(tiles):
    """With the shared expert's weights zero, doubling every route weight
    doubles the accumulator exactly: the coefficient enters before the
    second quantization, whose codes do not change under a power-of-two
    scale (scale and inverse double / halve exactly)."""
    L = _layer(seed=11, E=8, H=512, I=256, Is=128, T=3, k=2, tiles=tiles)
    L["shared_w2q"] = np.zeros_like(L["shared_w2q"])
    a1 = decode.fused_moe_decode(**L, return_acc=True)
    a2 = decode.fused_moe_decode(**{**L, "topk_weights": L["topk_weights"] * 2}, return_acc=True)
    np.testing.assert_array_equal(a2, 2 * a1)
    a3 = decode.fused_moe_decode(**L, routed_scale=2.0, return_acc=True)
    np.testing.assert_array_equal(a3, 2 * a1)
    assert np.abs(a1).max() > 0


def test_shared_expert_is_a_routed_expert_of_weight_one():
    """The shared expert runs the routed recipe with coefficient 1
    (ungated): moving it into the routed set as an expert of weight 1.0,
    with zero shared weights, gives the same accumulator bit for bit."""
    L = _layer(seed=13, E=6, H=512, I=256, Is=256, T=4, k=2)
    L["shared_gate"] = None
    ref = decode.fused_moe_decode(**{**L, "topk_weights": np.zeros_like(L["topk_weights"])}, return_acc=True)
    E = L["w1q"].shape[0]
    moved = dict(L)
    moved["w1q"] = np.concatenate([L["w1q"], L["shared_w1q"][None]])
    moved["w1s"] = np.concatenate([L["w1s"], L["shared_w1s"][None]])
    moved["w2q"] = np.concatenate([L["w2q"], L["shared_w2q"][None]])
    moved["w2s"] = np.concatenate([L["w2s"], L["shared_w2s"][None]])
    moved["shared_w2q"] = np.zeros_like(L["shared_w2q"])
    moved["topk_ids"] = np.full((4, 1), E, np.int32)
    moved["topk_weights"] = np.ones((4, 1), np.float32)
    np.testing.assert_array_equal(decode.fused_moe_decode(**moved, return_acc=True), ref)


def test_route_coefficients_sum_duplicates_and_round_weights():
    """`:639-646`: bf16-rounded weights, times routed_scale, summed over
    routes naming the same expert; ids outside [0, E) select nothing."""
    tw = np.array([[0.1, 0.2, 0.3], [0.5, 0.25, 1.0]], np.float32)
    ids = np.array([[2, 2, 0], [1, -1, 7]], np.int32)
    c = decode.route_coefficients(tw, ids, 4, routed_scale=2.0)
    b = _bf(tw)
    assert c[0, 2] == np.float32(b[0, 0] * 2) + np.float32(b[0, 1] * 2)
    assert c[0, 0] == np.float32(b[0, 2] * 2) and c[0, 1] == 0 and c[0, 3] == 0
    assert c[1, 1] == 1.0 and c[1].sum() == 1.0
    assert b[0, 0] != np.float32(0.1)  # the bf16 rounding matters here
