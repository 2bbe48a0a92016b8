"""The reference's runtime weight layouts at the op functions (host side, no
GPU): the e8m0 inverse, the fp4 K-major -> N-major repack, block sizes and
layout recognition (`qmoe/layers/ref_layout.py`)."""

import numpy as np
import pytest
import torch

from oracle import codecs
from qmoe.layers import ref_layout as rl


def test_e8m0_inverse_of_the_reference_decoding_for_every_byte():
    """f32 2^(b - 127) (the reference's ldexp decoding: b = 0 the subnormal
    2^-127, b = 255 +inf) maps back to every byte b."""
    b = np.arange(256, dtype=np.uint8)
    with np.errstate(over="ignore"):
        f = codecs.e8m0_decode(b)
    got = rl.f32_to_e8m0_exact(torch.from_numpy(f), "t").numpy()
    np.testing.assert_array_equal(got, b)


@pytest.mark.parametrize("v", [0.0, 3.0, -2.0, 0.75, float("nan")])
def test_e8m0_inverse_refuses_other_values(v):
    with pytest.raises(ValueError, match="e8m0"):
        rl.f32_to_e8m0_exact(torch.tensor([1.0, v], dtype=torch.float32), "t")


@pytest.mark.parametrize("shape", [(6, 20), (3, 4, 64)])
def test_fp4_kmajor_repack(shape):
    """K-major packing (two codes per byte along N, even n low) -> the
    checkpoint's N-major packing (two per byte along K, even k low): the
    oracle's unpack of the result equals the transposed code matrix."""
    rng = np.random.default_rng(sum(shape))
    *lead, n, k = shape
    codes = rng.integers(0, 16, (*lead, n, k), dtype=np.uint8)
    km = codecs.pack_fp4(np.swapaxes(codes, -1, -2).copy())  # [..., K, N/2]
    got = rl.fp4_kmajor_to_nmajor(torch.from_numpy(km)).numpy()
    np.testing.assert_array_equal(codecs.unpack_fp4(got), codes)
    np.testing.assert_array_equal(got, codecs.pack_fp4(codes))


def test_block_size_and_scale_transpose():
    s4 = torch.arange(2 * 4 * 6, dtype=torch.float32).reshape(2, 4, 1, 6)  # [E, K/B, 1, N]
    assert rl.block_of(s4, 512) == 128
    n = rl.scale_nmajor(s4)
    assert n.shape == (2, 6, 4) and torch.equal(n, s4[:, :, 0, :].transpose(1, 2))
    assert torch.equal(rl.scale_nmajor(s4[:, :, 0, :]), n)  # the rank-3 form
    with pytest.raises(ValueError):
        rl.block_of(s4, 510)


def test_moe_layout_recognition():
    E, H, I = 4, 256, 128
    f8 = torch.float8_e4m3fn
    ours13, ours2 = torch.empty(E, 2 * I, H, dtype=f8), torch.empty(E, H, I, dtype=f8)
    ref13, ref2 = torch.empty(E, H, 2 * I, dtype=f8), torch.empty(E, I, H, dtype=f8)
    # this package's scales: per channel [E, N], per (row, 128) [E, N, K/128], tiles [E, N/128, K/128]
    assert not rl.is_reference_moe_layout(H, ours13, ours2, torch.empty(E, 2 * I))
    assert not rl.is_reference_moe_layout(H, ours13, ours2, torch.empty(E, 2 * I, H // 128))
    assert not rl.is_reference_moe_layout(H, ours13, ours2, torch.empty(E, 2 * I // 128, H // 128))
    # the reference's: [E, K/B, 1, N] and [E, K/B, N]
    assert rl.is_reference_moe_layout(H, ref13, ref2, torch.empty(E, 1, 1, 2 * I))
    assert rl.is_reference_moe_layout(H, ref13, ref2, torch.empty(E, H // 128, 2 * I))
    # fp4 packed along N (reference) vs along K (this package)
    u8 = torch.uint8
    assert rl.is_reference_moe_layout(H, torch.empty(E, H, I, dtype=u8), torch.empty(E, I, H // 2, dtype=u8),
                                      torch.empty(E, H // 32, 2 * I))
    assert not rl.is_reference_moe_layout(H, torch.empty(E, 2 * I, H // 2, dtype=u8),
                                          torch.empty(E, H, I // 2, dtype=u8), torch.empty(E, 2 * I, H // 32))
    # bf16 without scales: by shape
    bf = torch.bfloat16
    assert rl.is_reference_moe_layout(H, torch.empty(E, H, 2 * I, dtype=bf), torch.empty(E, I, H, dtype=bf), None)
    assert not rl.is_reference_moe_layout(H, torch.empty(E, 2 * I, H, dtype=bf), torch.empty(E, H, I, dtype=bf),
                                          None)


def test_moe_weights_regimes_and_refusals():
    E, H, I = 2, 1024, 512
    f8 = torch.float8_e4m3fn
    w1 = torch.zeros(E, H, 2 * I, dtype=f8)
    w2 = torch.zeros(E, I, H, dtype=f8)
    # per channel: one K block
    *_, fmt = rl.moe_weights(H, w1, w2, torch.ones(E, 1, 1, 2 * I), torch.ones(E, 1, 1, H), None, None)
    assert fmt == "fp8"
    # B = 128: the W8A16 regime
    *_, fmt = rl.moe_weights(H, w1, w2, torch.ones(E, H // 128, 1, 2 * I), torch.ones(E, I // 128, 1, H), None, None)
    assert fmt == "fp8_w8a16"
    # B = 512: the quantized-activation regime
    *_, fmt = rl.moe_weights(H, w1, w2, torch.ones(E, H // 512, 1, 2 * I), torch.ones(E, I // 512, 1, H), None,
                             None)
    assert fmt == "fp8"
    with pytest.raises(NotImplementedError):
        rl.moe_weights(H, w1, w2, torch.ones(E, H // 256, 1, 2 * I), torch.ones(E, I // 64, 1, H), None, None)
    with pytest.raises(NotImplementedError, match="int4"):
        rl.moe_weights(H, torch.zeros(E, H // 8, 2 * I, dtype=torch.int32), w2, torch.ones(E, 8, 1, 2 * I),
                       torch.ones(E, 4, 1, H), None, None)


def test_repack_is_cached_per_weight_tensor():
    w = torch.arange(12, dtype=torch.uint8).reshape(3, 4)
    a = rl.nmajor_copy(w)
    assert rl.nmajor_copy(w) is a
    w.add_(1)  # an in-place change invalidates the copy
    b = rl.nmajor_copy(w)
    assert b is not a and torch.equal(b, w.t())


def test_repack_cache_under_inference_mode():
    """vLLM runs the forward under torch.inference_mode(): weights created
    there keep no version counter. The repack cache keys them on identity
    (nmajor_copy, fp4_linear, moe_weights), returns the same copy on the
    second call, and still follows in-place changes of ordinary tensors."""
    rng = np.random.default_rng(5)
    k, n = 64, 32
    with torch.inference_mode():
        w = torch.from_numpy(rng.integers(-100, 100, (k, n), dtype=np.int8))
        a = rl.nmajor_copy(w)
        assert a is rl.nmajor_copy(w)
        torch.testing.assert_close(a, w.t())
        codes = rng.integers(0, 16, (n, k), dtype=np.uint8)
        wq = torch.from_numpy(codecs.pack_fp4(codes.T.copy()))  # [K, N/2]
        ws = torch.full((1, k // 32, 1, n), 0.5, dtype=torch.float32)
        c, s = rl.fp4_linear(wq, ws, k)
        c2, s2 = rl.fp4_linear(wq, ws, k)
        assert c is c2 and s is s2
        np.testing.assert_array_equal(codecs.unpack_fp4(c.numpy()), codes)
        assert bool((s == 126).all())
        E, H, I = 2, 64, 32
        w1 = torch.from_numpy(rng.integers(-100, 100, (E, H, 2 * I), dtype=np.int8))
        w2 = torch.from_numpy(rng.integers(-100, 100, (E, I, H), dtype=np.int8))
        s1 = torch.ones((E, 1, 1, 2 * I), dtype=torch.float32)
        s2 = torch.ones((E, 1, 1, H), dtype=torch.float32)
        r1 = rl.moe_weights(H, w1, w2, s1, s2, None, None)
        r2 = rl.moe_weights(H, w1, w2, s1, s2, None, None)
        assert r1[0] is r2[0] and r1[1] is r2[1] and r1[-1] == "int8"
        torch.testing.assert_close(r1[0], w1.transpose(1, 2))
    # an ordinary tensor changed in place is repacked again
    v = torch.from_numpy(rng.integers(-100, 100, (k, n), dtype=np.int8))
    b = rl.nmajor_copy(v)
    v.add_(1)
    b2 = rl.nmajor_copy(v)
    assert b2 is not b
    torch.testing.assert_close(b2, v.t())
