"""The reference's runtime weight layouts at the op functions.

The reference's load transforms leave its weights K-major, the layout its
grouped matmul reads (`kernels/megablox/gmm_v2.py:1280-1443`, rhs ``[G, K,
N]``):

* ``quantized_matmul(x, w_q, w_s)`` (`layers/adapter/linear_common.py:
  162-185`): ``w_q`` a contiguous ``[n_in, n_out]`` tensor (flipped at
  load, `layers/adapter/quantization/fp8.py:1598-1617`);
* ``quantized_matmul_fp4(x, w_q, w_s)`` (`layers/adapter/linear_common.py:
  188-209, 242-255`): ``w_q`` native fp4 ``[n_in, n_out]`` stored as
  ``torch.float4_e2m1fn_x2`` (two codes per byte along n_out, the even one in
  the low nibble: a ``[n_in, n_out / 2]`` byte tensor) and ``w_s`` the fused
  float32 block scale ``[1, n_in / B, 1, n_out]``;
* ``fused_moe_gmm`` (`layers/adapter/fused_moe.py:241-293` ->
  `layers/core/fused_moe_gmm.py:592-728`): ``w1 [E, H, 2I]``, ``w2 [E, I,
  H]`` (1-byte codes, bf16, or native fp4 packed along N as above), scales
  ``[E, K / B, 1, N]`` float32 (or ``[E, K / B, N]``, which the reference
  expands at `fused_moe_gmm.py:631-636`), biases ``[E, 1, N]``.

This package's kernels read N-major weights (each output channel's K
contiguous: the checkpoint layout), so a reference-layout weight is
repacked once: the N-major copy is cached for the lifetime of the weight
tensor (keyed weakly on it and on its in-place version counter) and later
calls with the same tensor reuse it. The numeric regime follows the scale's
block size B as the reference's grouped matmul selects it
(`gmm_v2.py:242-273, 452-548`): fp4 blocks of 16 are NVFP4 (bf16 block
scales) and of 32 MXFP4 (the scales must then be powers of two, exactly
e8m0); 1-byte codes with B < 256 run the dequantize-before-matmul W8A16
regime (B = 128), and B >= 256 (or one block: per channel) the
quantized-activation regime.
"""

import weakref

import torch

FP4X2 = getattr(torch, "float4_e2m1fn_x2", None)

# id(weight tensor) -> (weak reference to it, {key: (version, converted)});
# the entry goes when the tensor does (tensors compare elementwise, so they
# cannot be WeakKeyDictionary keys)
_CACHE = {}


def _version_of(t: torch.Tensor):
    """The in-place version counter of `t`, or None for an inference tensor
    (created under ``torch.inference_mode()``, as vLLM's forward runs): such
    tensors keep no counter, so their cache entry is keyed on identity
    alone."""
    return None if t.is_inference() else t._version


def _cached(t: torch.Tensor, key, make):
    """`make()` once per (weight tensor, key, in-place version)."""
    tid = id(t)
    ent = _CACHE.get(tid)
    if ent is None or ent[0]() is not t:
        ent = (weakref.ref(t, lambda _r, tid=tid: _CACHE.pop(tid, None)), {})
        _CACHE[tid] = ent
    slot = ent[1]
    hit = slot.get(key)
    ver = _version_of(t)
    if hit is not None and hit[0] == ver:
        return hit[1]
    out = make()
    slot[key] = (ver, out)
    return out


def nmajor_copy(w_kn: torch.Tensor) -> torch.Tensor:
    """A K-major ``[n_in, n_out]`` 1-byte / bf16 weight -> its N-major
    ``[n_out, n_in]`` copy, made once per weight tensor."""
    return _cached(w_kn, "nmajor2d", lambda: w_kn.t().contiguous())


def as_bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def fp4_kmajor_to_nmajor(w: torch.Tensor) -> torch.Tensor:
    """Packed e2m1 ``[..., K, N/2]`` (two codes per byte along N) -> N-major
    ``[..., N, K/2]`` (two codes per byte along K, even k in the low nibble)."""
    b = as_bytes(w)
    codes = torch.stack((b & 0xF, b >> 4), dim=-1).flatten(-2)  # [..., K, N]
    codes = codes.transpose(-1, -2)  # [..., N, K]
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()


def block_of(w_s: torch.Tensor, k: int) -> int:
    """Block size B of a ``[..., K/B, 1, N]`` / ``[..., K/B, N]`` scale."""
    nb = w_s.shape[-3] if w_s.dim() >= 4 else w_s.shape[-2]
    if nb <= 0 or k % nb:
        raise ValueError(f"scale with {nb} K blocks does not divide K = {k}")
    return k // nb


def scale_nmajor(w_s: torch.Tensor) -> torch.Tensor:
    """``[..., K/B, 1, N]`` or ``[..., K/B, N]`` float32 -> ``[..., N, K/B]``."""
    s = w_s.squeeze(-2) if w_s.dim() >= 4 else w_s
    return s.transpose(-1, -2).to(torch.float32).contiguous()


def f32_to_e8m0_exact(s: torch.Tensor, what: str) -> torch.Tensor:
    """float32 scales that are e8m0 values -> e8m0 bytes: 2^(b - 127) for b in
    1..254 (normal powers of two), 2^-127 (the float32 subnormal) for b = 0,
    +inf for b = 255 -- the inverse of `layers/core/quantization.py:105-128`'s
    float32 ldexp decoding. Any other value is refused."""
    bits = s.contiguous().view(torch.int32)
    exp = (bits >> 23) & 0xFF
    normal = ((bits & 0x7FFFFF) == 0) & (exp > 0) & (exp < 255) & (bits >= 0)
    sub = bits == 0x00400000
    inf = bits == 0x7F800000
    if not bool((normal | sub | inf).all()):
        raise ValueError(f"{what}: block-32 fp4 scales must be e8m0 values (powers of two); "
                         "use block-16 scales for NVFP4 weights")
    return torch.where(sub, torch.zeros_like(exp), exp).to(torch.uint8)


def fp4_linear(w_q: torch.Tensor, w_s: torch.Tensor, k: int):
    """Reference-layout dense fp4 weight + ``[1, K/B, 1, N]`` scale -> this
    package's (codes ``[N, K/2]``, scales) with the scale dtype naming the
    format: bf16 ``[N, K/16]`` (NVFP4) or e8m0 bytes ``[N, K/32]`` (MXFP4)."""
    if w_s.dim() != 4 or w_s.shape[0] != 1 or w_s.shape[2] != 1:
        raise ValueError(f"quantized_matmul_fp4: reference scale must be [1, K/B, 1, N], got {tuple(w_s.shape)}")
    n_out = w_s.shape[-1]
    if w_q.dim() != 2 or w_q.shape[0] != k or w_q.shape[1] * 2 != n_out:
        raise ValueError(f"quantized_matmul_fp4: reference weight must be fp4 [n_in={k}, n_out={n_out}] "
                         f"(bytes [{k}, {n_out // 2}]), got {tuple(w_q.shape)} {w_q.dtype}")
    blk = block_of(w_s, k)
    if blk not in (16, 32):
        raise NotImplementedError(f"quantized_matmul_fp4: fp4 blocks of {blk} are not supported (16 or 32)")
    codes = _cached(w_q, "fp4_nmajor", lambda: fp4_kmajor_to_nmajor(w_q))
    if blk == 16:
        sc = _cached(w_s, "nv_bf16", lambda: scale_nmajor(w_s)[0].to(torch.bfloat16).contiguous())
    else:
        sc = _cached(w_s, "mx_e8m0", lambda: f32_to_e8m0_exact(scale_nmajor(w_s)[0], "quantized_matmul_fp4"))
    return codes, sc


def is_reference_moe_layout(hidden: int, w1: torch.Tensor, w2: torch.Tensor, w1_scale) -> bool:
    """Whether fused_moe_gmm's weights are in the reference's K-major layout:
    a rank-4 ``[E, K/B, 1, N]`` scale, a rank-3 scale whose last axis is N (a
    rank-3 scale of this package is ``[E, N, K/B]`` or ``[E, N/128, K/128]``),
    or unscaled weights shaped ``[E, H, 2I]`` / ``[E, I, H]`` where this
    package's ``[E, 2I, H]`` / ``[E, H, I]`` reading does not fit."""
    if w1_scale is not None:
        if w1_scale.dim() == 4:
            return True
        if w1_scale.dim() == 3:
            n_last = w1.shape[-1] * (2 if (w1.dtype == torch.uint8 or w1.dtype == FP4X2) else 1)
            return w1_scale.shape[-1] == n_last
        return False
    ours = w1.shape[-1] == hidden and w2.shape[1] == hidden
    ref = w1.shape[1] == hidden and w2.shape[-1] == hidden
    return ref and not ours


def moe_weights(hidden: int, w1, w2, w1_scale, w2_scale, w1_bias, w2_bias):
    """Reference-layout MoE weights -> this package's (w1 ``[E, 2I, H...]``,
    w2, scales, biases, format), repacked once per weight tensor."""
    E = w1.shape[0]
    fp4 = w1.dtype == torch.uint8 or w1.dtype == FP4X2
    if w1.dtype == torch.int32 or str(w1.dtype) == "torch.uint32":
        raise NotImplementedError("fused_moe_gmm: reference-layout packed-int4 weights are not accepted; pass the "
                                  "compressed-tensors checkpoint form (int32 carriers [E, N, K/8], bf16 group "
                                  "scales [E, N, K/group]) with rhs_quant_dtype=int4")
    k1 = w1.shape[1]  # H
    k2 = w2.shape[1]  # I
    if fp4:
        if w1_scale is None or w2_scale is None:
            raise ValueError("fused_moe_gmm: fp4 weights need block scales [E, K/B, 1, N]")
        b1, b2 = block_of(w1_scale, k1), block_of(w2_scale, k2)
        if b1 != b2 or b1 not in (16, 32):
            raise NotImplementedError(f"fused_moe_gmm: fp4 blocks of {b1} / {b2} are not supported (16 or 32)")
        c1 = _cached(w1, "fp4_nmajor", lambda: fp4_kmajor_to_nmajor(w1))
        c2 = _cached(w2, "fp4_nmajor", lambda: fp4_kmajor_to_nmajor(w2))
        if b1 == 16:
            s1 = _cached(w1_scale, "nv_bf16", lambda: scale_nmajor(w1_scale).to(torch.bfloat16).contiguous())
            s2 = _cached(w2_scale, "nv_bf16", lambda: scale_nmajor(w2_scale).to(torch.bfloat16).contiguous())
            fmt = "nvfp4"
        else:
            s1 = _cached(w1_scale, "mx_e8m0", lambda: f32_to_e8m0_exact(scale_nmajor(w1_scale), "fused_moe_gmm w1"))
            s2 = _cached(w2_scale, "mx_e8m0", lambda: f32_to_e8m0_exact(scale_nmajor(w2_scale), "fused_moe_gmm w2"))
            fmt = "mxfp4"
    else:
        c1 = _cached(w1, "nmajor", lambda: w1.transpose(1, 2).contiguous())
        c2 = _cached(w2, "nmajor", lambda: w2.transpose(1, 2).contiguous())
        if w1.dtype == torch.bfloat16:
            if w1_scale is not None or w2_scale is not None:
                raise ValueError("fused_moe_gmm: bf16 weights take no scales")
            s1 = s2 = None
            fmt = "bf16"
        elif w1.dtype in (torch.float8_e4m3fn, torch.int8, torch.float8_e5m2):
            if w1_scale is None or w2_scale is None:
                raise ValueError("fused_moe_gmm: 1-byte weights need scales [E, K/B, 1, N]")
            b1, b2 = block_of(w1_scale, k1), block_of(w2_scale, k2)
            q = {torch.int8: "int8", torch.float8_e5m2: "e5m2"}.get(w1.dtype, "fp8")
            s1n = _cached(w1_scale, "nmajor", lambda: scale_nmajor(w1_scale))  # [E, N, K/B]
            s2n = _cached(w2_scale, "nmajor", lambda: scale_nmajor(w2_scale))
            if b1 == k1 and b2 == k2:  # one block: per channel
                s1, s2, fmt = s1n[..., 0].contiguous(), s2n[..., 0].contiguous(), q
            elif b1 == 128 and b2 == 128 and q == "fp8":  # B < 256: W8A16 regime
                s1, s2, fmt = s1n, s2n, "fp8_w8a16"
            elif b1 >= 512 and b2 >= 512 and (b1 & (b1 - 1)) == 0 and (b2 & (b2 - 1)) == 0:
                s1, s2, fmt = s1n, s2n, q  # per (row, B) blocks, quantized-activation regime
            else:
                raise NotImplementedError(f"fused_moe_gmm: {q} scale blocks of {b1} / {b2} are not supported "
                                          "(per channel, 128 for fp8, or a power of two >= 512)")
        else:
            raise ValueError(f"fused_moe_gmm: unsupported reference-layout weight dtype {w1.dtype}")
    b1n = None if w1_bias is None else _cached(w1_bias, "bias", lambda: w1_bias.reshape(E, -1).float().contiguous())
    b2n = None if w2_bias is None else _cached(w2_bias, "bias", lambda: w2_bias.reshape(E, -1).float().contiguous())
    return c1, c2, s1, s2, b1n, b2n, fmt
