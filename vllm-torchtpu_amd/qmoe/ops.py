"""Torch-facing wrappers of the qmoe C ABI.

Every function here takes device tensors (HIP), validates shapes / dtypes /
layouts on the host, and launches the HIP kernels on the current stream via
`_capi`. There is no CPU path: a CPU tensor is a ValueError.
"""

import ctypes
import math

import torch

from qmoe import _capi
from qmoe._capi import GemmDesc, check, lib

FP8 = torch.float8_e4m3fn

_ACT_CODES = {
    None: (_capi.ACT_NONE, 0.0, 0.0),
    "silu": (_capi.ACT_SILU, 0.0, 0.0),
    "swigluoai": (_capi.ACT_SWIGLUOAI, 1.702, 7.0),
    "gelu": (_capi.ACT_GELU_TANH, 0.0, 0.0),  # jax.nn.gelu defaults to tanh form
    "gelu_tanh": (_capi.ACT_GELU_TANH, 0.0, 0.0),
    "silu_and_mul_with_clamp": (_capi.ACT_SILU_CLAMP, 10.0, 0.0),
}


def act_code(activation):
    """Activation string (`kernels/megablox/gmm_v2.py:101-122`) -> code."""
    if activation in _ACT_CODES:
        return _ACT_CODES[activation]
    if isinstance(activation, str) and activation.startswith("situ:"):
        _, beta, lin = activation.split(":")
        return _capi.ACT_SITU, float(beta), (-1.0 if lin == "none" else float(lin))
    raise NotImplementedError(f"Unsupported activation function: {activation}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _require_gpu(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"qmoe kernels need device tensors, got a {t.device} tensor")


def _bytes_view(t):
    """1-byte code tensors (float8 / int8 / uint8 / packed fp4) as uint8."""
    if t.element_size() != 1:
        raise ValueError(f"expected a 1-byte code tensor, got {t.dtype}")
    return t.view(torch.uint8)


# ---------------------------------------------------------------- workspace


def _workspace(dev, nbytes):
    """Scratch for one call (split-K partial sums, the fused decode op's
    dispatch and intermediates), taken from torch's caching allocator on the
    current stream. The allocator keeps a block on the stream it was made
    on until the work queued there has used it, and a HIP graph captured
    around the call owns its block for the graph's lifetime, so concurrent
    streams never share bytes and a replay never reaches freed memory. The
    kernels write every byte they read (the decode op clears its own
    block-maximum table in its first launch), so nothing is cleared here."""
    if nbytes <= 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=dev), nbytes


# ---------------------------------------------------------------- row quant


def row_quant(x, qdtype="fp8", block=None, mode="runtime"):
    """Quantize rows of ``x`` ([M, K] bf16, or f32 for mode="load").

    mode "runtime": `kernels/quantized_matmul/util.py:294-318` semantics
    (scale = absmax / qmax; fp8 in f32, int8 in bf16 arithmetic; zero scale
    -> 1). mode "load": `layers/core/quantization.py:232-318` (reciprocal
    multiply; zero rows keep scale 0). mode "gmm": the grouped matmul's
    quantized-lhs regime, `kernels/megablox/gmm_v2.py:508-536` (per (row,
    512 columns), bf16 arithmetic, fp8 RNE / int8 truncated codes; block is
    always 512). qdtype "fp8" (e4m3fn), "int8" or "e5m2" (one scale per row,
    modes "runtime" and "load"). Returns (codes [M, K] float8_e4m3fn, int8 or
    float8_e5m2, scales f32 [M], [M, K/128] or [M, ceil(K/512)]).
    """
    _require_gpu(x)
    if x.dim() != 2:
        raise ValueError(f"row_quant expects a 2-D tensor, got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    M, K = x.shape
    in_f32 = x.dtype == torch.float32
    if not in_f32 and x.dtype != torch.bfloat16:
        raise ValueError(f"row_quant expects bf16 (or f32 at load time), got {x.dtype}")
    qd = {"fp8": 0, "int8": 1, "e5m2": 2}[qdtype]
    md = {"runtime": 0, "load": 1, "gmm": 2}[mode]
    blk = 512 if md == 2 else (0 if block is None else int(block))
    if qd == 2 and blk:
        raise ValueError("row_quant: e5m2 codes take one scale per row (no blocks, no gmm mode)")
    q = torch.empty((M, K), dtype=(FP8, torch.int8, torch.float8_e5m2)[qd], device=x.device)
    ns = 1 if blk == 0 else (K + blk - 1) // blk
    s = torch.empty((M, ns), dtype=torch.float32, device=x.device)
    if M:
        check(lib.qmoe_row_quant(_ptr(x), x.stride(0), int(in_f32), M, K, qd, md, blk, _ptr(q), K,
                                 _ptr(s), ns, _stream(x.device)), "row_quant")
    return q, (s[:, 0] if blk == 0 else s)


def mx_quant(x, k_pad=None, codes=True, dequantized=False):
    """MX activation quantization of bf16 rows ``x`` [M, K] (K % 32 == 0):
    the reference's ue8m0 block rule (`layers/core/quantization.py:232-318`,
    scale = amax * f32(1/6) snapped up to a power of two) with its e2m1
    encoder (`compressed_tensors_moe/utils.py:167-183`), per 32 columns.

    ``codes``: returns e2m1 codes packed two per byte (low nibble = even
    column) ``[M, Kp/2]`` uint8 and e8m0 bytes ``[M, Kp/32]`` uint8, columns
    K..Kp-1 zero (``k_pad`` = Kp, a multiple of 32, default K).
    ``dequantized``: also (or only, with ``codes=False``) the quantized values
    as bf16 ``[M, K]`` (exact). Returns the requested tensors in that order.
    """
    _require_gpu(x)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise ValueError(f"mx_quant expects bf16 [M, K], got {x.dtype} {tuple(x.shape)}")
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    M, K = x.shape
    kp = K if k_pad is None else int(k_pad)
    if K % 32 or kp % 32 or kp < K:
        raise ValueError(f"mx_quant needs K ({K}) and the padded K ({kp}) to be multiples of 32, K <= padded K")
    if not codes and not dequantized:
        raise ValueError("mx_quant: nothing requested")
    dev = x.device
    q = torch.empty((M, kp // 2), dtype=torch.uint8, device=dev) if codes else None
    sc = torch.empty((M, kp // 32), dtype=torch.uint8, device=dev) if codes else None
    xq = torch.empty((M, K), dtype=torch.bfloat16, device=dev) if dequantized else None
    if M:
        check(lib.qmoe_mx_quant(_ptr(x), x.stride(0), M, K, kp, _ptr(q) if codes else None, kp // 2,
                                _ptr(sc) if codes else None, kp // 32, _ptr(xq) if dequantized else None, K,
                                _stream(dev)), "mx_quant")
    out = ((q, sc) if codes else ()) + ((xq,) if dequantized else ())
    return out if len(out) > 1 else out[0]


# ---------------------------------------------------------------- GEMM


def gemm(kind, a, w, **kw):
    """Run one (grouped) quantized GEMM through `qmoe_gemm` (arguments as
    `gemm_desc`); the split-K workspace is allocated for the call on the
    current stream. Returns ``out`` ([M, N or N/2] bf16 unless given)."""
    d, out = gemm_desc(kind, a, w, **kw)
    dev = a.device
    need = ctypes.c_int64(0)
    check(lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(need)), "gemm (plan)")
    if _plan_log is not None:
        _plan_log.append(plan_of_desc(d))
    ws_t, ws_n = _workspace(dev, need.value)
    check(lib.qmoe_gemm(ctypes.byref(d), _ptr(ws_t), ws_n, _stream(dev)), "gemm")
    return out


def gemm_desc(kind, a, w, *, a_scale=None, w_scale=None, bias=None, wfmt=0, ws_bn=1,
              group_offs=None, active=None, num_active=None, slots=1, max_rows=None, a_rows=None,
              activation=None, row_weight=None, out=None, y_rows=None, M=None):
    """Checked `qmoe_gemm_desc` of one (grouped) quantized GEMM, and its
    output tensor (allocated here unless ``out`` is given).

    a        : [rows, K] activation codes (1 byte) or bf16; W4A4_MX: packed e2m1 [rows, K/2]
               with e8m0 bytes [rows, K/32] in ``a_scale``
    w        : [G, N, K] / [N, K] weights (1 byte codes, packed e2m1 [.., K/2], bf16)
    w_scale  : per-channel f32 [G, N] | block f32 [G, N/bn, K/128] | e8m0 u8 [G, N, K/32]
               | NVFP4 bf16 [G, N, K/16] | INT4 bf16 [G, N, K/group] (group 32, 64 or 128)
    """
    _require_gpu(a, w)
    dev = a.device
    if w.dim() == 2:
        w = w.unsqueeze(0)
    G, N, wcols = w.shape
    # rows may be padded (a row stride above the row length, 16-byte multiples)
    if a.stride(-1) != 1 or w.stride(-1) != 1 or w.stride(1) < wcols or w.stride(0) < N * w.stride(1):
        raise ValueError("qmoe gemm needs K-contiguous activations and N-major [G, N, K] weights")
    abf16 = kind in (_capi.W8A16_PC, _capi.W4A16_MX, _capi.W16A16, _capi.W4A16_NV, _capi.W4A16_I4,
                     _capi.W8A16_BLK, _capi.W8A8_PC_DYN)
    K = a.shape[1] * (2 if kind == _capi.W4A4_MX else 1)
    if kind == _capi.W4A4_MX and (a.dtype != torch.uint8 or a_scale is None or a_scale.dtype != torch.uint8
                                  or a_scale.dim() != 2 or a_scale.shape[1] * 32 < K):
        raise ValueError("W4A4_MX takes packed e2m1 activations [M, K/2] uint8 with e8m0 bytes [M, K/32]")
    if kind in (_capi.W4A16_MX, _capi.W4A16_NV, _capi.W4A16_I4, _capi.W4A4_MX):
        if wcols * 2 != K:
            raise ValueError(f"packed e2m1 weight has {wcols} bytes per row, expected K/2 = {K // 2}")
    elif wcols != K:
        raise ValueError(f"Input hidden dim {K} must match weight hidden dim {wcols}.")
    if abf16 and a.dtype != torch.bfloat16:
        raise ValueError(f"this kind takes bf16 activations, got {a.dtype}")
    if M is None:
        M = a.shape[0] if a_rows is None else a_rows.shape[0]
    act, p0, p1 = act_code(activation)
    nout = N // 2 if act != _capi.ACT_NONE else N
    if out is None:
        out = torch.empty((M, nout), dtype=torch.bfloat16, device=dev)
    d = GemmDesc()
    d.kind = kind
    d.wfmt = wfmt
    d.a = a.data_ptr()
    d.lda = a.stride(0)
    if a_scale is not None:
        d.a_scale = a_scale.data_ptr()
        d.lds_a = a_scale.stride(0) if a_scale.dim() == 2 else 1
    d.a_rows = a_rows.data_ptr() if a_rows is not None else None
    d.w = w.data_ptr()
    d.ldw = w.stride(1) * w.element_size()
    d.w_gstride = w.stride(0) * w.element_size()
    if w_scale is not None:
        ws = w_scale
        if kind in (_capi.W8A8_PC, _capi.W8A16_PC, _capi.W8A8_PC_DYN) or (kind == _capi.W8A8_GMM and
                                                                           ws.numel() == G * N):
            ws = ws.reshape(G, N)
            d.ldws, d.ws_gstride = 1, ws.stride(0)
        else:
            if ws.dim() == 2:
                ws = ws.unsqueeze(0)
            if kind == _capi.W4A16_NV and (ws.dtype != torch.bfloat16 or ws.shape[-1] * 16 != K):
                raise ValueError(f"NVFP4 weight scales are bf16 [G, N, K/16], got {ws.dtype} {tuple(ws.shape)}")
            if kind == _capi.W4A16_I4:
                grp = K // ws.shape[-1] if ws.shape[-1] else 0
                if ws.dtype != torch.bfloat16 or grp not in (32, 64, 128) or grp * ws.shape[-1] != K:
                    raise ValueError(f"INT4 weight scales are bf16 [G, N, K/group] with group 32, 64 or 128, "
                                     f"got {ws.dtype} {tuple(ws.shape)} for K={K}")
                d.wq_group = grp
            d.ldws, d.ws_gstride = ws.stride(1), ws.stride(0)
        d.w_scale = ws.data_ptr()
    d.ws_bn = ws_bn
    if bias is not None:
        b = bias.reshape(G, N)
        if b.dtype != torch.float32:
            raise ValueError("bias must be float32 [G, N]")
        d.bias, d.bias_gstride = b.data_ptr(), b.stride(0)
    d.group_offs = group_offs.data_ptr() if group_offs is not None else None
    d.active = active.data_ptr() if active is not None else None
    d.num_active = num_active.data_ptr() if num_active is not None else None
    d.slots = slots
    d.max_rows = max_rows if max_rows is not None else M
    d.M, d.N, d.K = M, N, K
    d.act, d.act_p0, d.act_p1 = act, p0, p1
    d.row_weight = row_weight.data_ptr() if row_weight is not None else None
    d.y = out.data_ptr()
    d.ldy = out.stride(0)
    d.y_rows = y_rows.data_ptr() if y_rows is not None else None
    return d, out


# ---------------------------------------------------------------- kernel plans

PATH_NAMES = ("stream", "tiled_1b", "tiled_4b", "tiled_generic", "stream_passes", "tiled_1b_persistent",
              "tiled_mx_persistent", "tiled_mx", "stream_dyn", "tiled_1b_n128", "stream_rows")

_plan_log = None


def plan_of_desc(d):
    """(kind, wfmt, fused activation, grouped, path name, token rows per
    tile, K split) that `qmoe_gemm` picks for the descriptor (host-side
    `qmoe_gemm_plan`)."""
    path, tile, ks = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_int32(0)
    check(lib.qmoe_gemm_plan(ctypes.byref(d), ctypes.byref(path), ctypes.byref(tile), ctypes.byref(ks)),
          "gemm_plan")
    return (int(d.kind), int(d.wfmt), int(d.act != _capi.ACT_NONE), int(bool(d.group_offs)),
            PATH_NAMES[path.value], int(tile.value), int(ks.value))


class record_plans:
    """Context manager collecting the plan of every `gemm` call made inside
    it (a list of `plan_of_desc` tuples)."""

    def __enter__(self):
        global _plan_log
        self._prev = _plan_log
        _plan_log = self.plans = []
        return self.plans

    def __exit__(self, *exc):
        global _plan_log
        _plan_log = self._prev
        if self._prev is not None:
            self._prev.extend(self.plans)
        return False


def plan_for_shape(kind, M, N, K, *, wfmt=0, activation=None, experts=0, max_rows=None, ws_bn=1,
                   wq_group=0, lda=None):
    """The plan `qmoe_gemm` makes for a problem of this shape, from a
    descriptor with placeholder (aligned, never dereferenced) addresses and
    contiguous strides: dense when ``experts == 0``, else grouped over
    ``experts`` groups with an active list, ``max_rows`` rows at most per
    group (the MoE layer passes the token count). Needs no GPU."""
    w4 = kind in (_capi.W4A16_MX, _capi.W4A16_NV, _capi.W4A16_I4, _capi.W4A4_MX)
    act, p0, p1 = act_code(activation)
    base = 1 << 24
    d = GemmDesc()
    d.kind, d.wfmt = kind, wfmt
    d.a = d.w = d.y = d.w_scale = d.a_scale = base
    d.lda = lda if lda is not None else (K // 2 if kind == _capi.W4A4_MX else K)
    d.lds_a = K // 128 if kind == _capi.W8A8_BLK else ((K + 511) // 512 if kind == _capi.W8A8_GMM else 1)
    if kind == _capi.W4A4_MX:
        d.lds_a = K // 32
    ldw = K // 2 if w4 else (2 * K if kind == _capi.W16A16 else K)
    d.ldw, d.w_gstride = ldw, ldw * N
    if kind in (_capi.W8A8_BLK, _capi.W8A16_BLK):
        d.ldws = K // 128
    elif kind in (_capi.W4A16_MX, _capi.W4A4_MX):
        d.ldws = K // 32
    elif kind == _capi.W4A16_NV:
        d.ldws = K // 16
    elif kind == _capi.W4A16_I4:
        d.ldws = K // wq_group
    else:
        d.ldws = 1
    d.ws_gstride = d.ldws * (N // ws_bn if kind in (_capi.W8A8_BLK, _capi.W8A16_BLK) else N)
    d.ws_bn, d.wq_group = ws_bn, wq_group
    if experts:
        d.group_offs = d.active = d.num_active = base
        d.slots = experts
    else:
        d.slots = 1
    d.max_rows = max_rows if max_rows is not None else M
    d.M, d.N, d.K = M, N, K
    d.act, d.act_p0, d.act_p1 = act, p0, p1
    d.ldy = N // 2 if act != _capi.ACT_NONE else N
    return plan_of_desc(d)


# ---------------------------------------------------------------- MoE


_SCORING = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2, "none": 3}


def moe_route(router_logits, topk, scoring_func="softmax", renormalize=True, bias=None,
              routed_scaling_factor=1.0, num_expert_group=1, topk_group=1, weights_f32=False):
    """Router on the GPU: (bf16 (or f32) weights [T, k], int32 ids [T, k]).

    scoring_func "none" takes the input as scores (rowmax top-k only)."""
    _require_gpu(router_logits, bias)
    if scoring_func not in _SCORING:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    x = router_logits.reshape(-1, router_logits.shape[-1])
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    T, E = x.shape
    if topk > E:
        raise ValueError(f"topk k={topk} exceeds the expert count {E}")
    w = torch.empty((T, topk), dtype=torch.float32 if weights_f32 else torch.bfloat16,
                    device=x.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=x.device)
    b = bias.float().contiguous() if bias is not None else None
    check(lib.qmoe_moe_route(_ptr(x), int(x.dtype == torch.float32), T, E, topk,
                             _SCORING[scoring_func], _ptr(b), int(bool(renormalize)),
                             float(routed_scaling_factor), int(num_expert_group or 1),
                             int(topk_group or 1), _ptr(w), int(bool(weights_f32)), _ptr(ids),
                             _stream(x.device)),
          "moe_route")
    return w, ids


def _dispatch_meta(nf, num_experts, dev):
    i32 = dict(dtype=torch.int32, device=dev)
    return dict(
        sorted_idx=torch.empty(nf, **i32),
        revert=torch.empty(nf, **i32),
        token_sorted=torch.empty(nf, **i32),
        group_offs=torch.empty(num_experts + 1, **i32),
        active=torch.empty(max(1, min(num_experts, nf)), **i32),
        num_active=torch.empty(1, **i32),
        sorted_weight=torch.empty(nf, dtype=torch.bfloat16, device=dev),
    )


ROUTE_DISPATCH_MAX_TOKENS = 16
ROUTE_DISPATCH_MAX_ROUTES = 64


def moe_route_dispatch(router_logits, topk, scoring_func="softmax", renormalize=True, bias=None,
                       routed_scaling_factor=1.0, num_expert_group=1, topk_group=1, skip_padded_tokens=False):
    """Routing + dispatch of a decode step in one launch (1 <= T <= 16,
    T * topk <= 64): (bf16 weights [T, k], int32 ids [T, k], dispatch
    metadata as returned by `moe_dispatch`)."""
    _require_gpu(router_logits, bias)
    if scoring_func not in _SCORING:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    x = router_logits.reshape(-1, router_logits.shape[-1])
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    T, E = x.shape
    if not (1 <= T <= ROUTE_DISPATCH_MAX_TOKENS and T * topk <= ROUTE_DISPATCH_MAX_ROUTES):
        raise ValueError(f"route + dispatch takes 1..16 tokens and at most 64 routes, got T={T}, k={topk}")
    dev = x.device
    w = torch.empty((T, topk), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((T, topk), dtype=torch.int32, device=dev)
    meta = _dispatch_meta(T * topk, E, dev)
    b = bias.float().contiguous() if bias is not None else None
    check(lib.qmoe_moe_route_dispatch(_ptr(x), int(x.dtype == torch.float32), T, E, topk, _SCORING[scoring_func],
                                      _ptr(b), int(bool(renormalize)), float(routed_scaling_factor),
                                      int(num_expert_group or 1), int(topk_group or 1), _ptr(w), _ptr(ids),
                                      int(bool(skip_padded_tokens)), _ptr(meta["sorted_idx"]),
                                      _ptr(meta["revert"]), _ptr(meta["token_sorted"]),
                                      _ptr(meta["group_offs"]), _ptr(meta["active"]),
                                      _ptr(meta["num_active"]), _ptr(meta["sorted_weight"]), _stream(dev)),
          "moe_route_dispatch")
    return w, ids, meta


def moe_route_hash(router_logits, topk, hash_indices_table, input_ids, scoring_func="softmax", renormalize=True,
                   routed_scaling_factor=1.0):
    """DeepSeek-V4 hash routing on the GPU: (bf16 weights [T, k], int32 ids
    [T, k]) with ids = hash_indices_table[input_ids]."""
    _require_gpu(router_logits, hash_indices_table, input_ids)
    if scoring_func not in _SCORING:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    x = router_logits.reshape(-1, router_logits.shape[-1])
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    T, E = x.shape
    table = hash_indices_table.to(torch.int32).contiguous()
    if table.dim() != 2 or table.shape[1] != topk:
        raise ValueError(f"hash_indices_table must be [vocab, {topk}], got {tuple(table.shape)}")
    ids_in = input_ids.reshape(-1)
    if ids_in.numel() != T:
        raise ValueError(f"{ids_in.numel()} input ids for {T} tokens")
    if ids_in.dtype not in (torch.int32, torch.int64):
        ids_in = ids_in.to(torch.int64)
    ids_in = ids_in.contiguous()
    w = torch.empty((T, topk), dtype=torch.bfloat16, device=x.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=x.device)
    check(lib.qmoe_moe_route_hash(_ptr(x), int(x.dtype == torch.float32), T, E, topk, _SCORING[scoring_func],
                                  _ptr(table), table.shape[0], _ptr(ids_in), int(ids_in.dtype == torch.int64),
                                  int(bool(renormalize)), float(routed_scaling_factor), _ptr(w), _ptr(ids),
                                  _stream(x.device)), "moe_route_hash")
    return w, ids


def moe_dispatch(topk_ids, topk_weights, num_experts, skip_padded_tokens=False):
    """Permutation metadata (see include/qmoe.h `qmoe_moe_dispatch`)."""
    _require_gpu(topk_ids, topk_weights)
    T, k = topk_ids.shape
    dev = topk_ids.device
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.bfloat16).contiguous()
    nf = T * k
    meta = _dispatch_meta(nf, num_experts, dev)
    check(lib.qmoe_moe_dispatch(_ptr(ids), _ptr(wts), T, k, num_experts, int(bool(skip_padded_tokens)),
                                _ptr(meta["sorted_idx"]), _ptr(meta["revert"]),
                                _ptr(meta["token_sorted"]), _ptr(meta["group_offs"]),
                                _ptr(meta["active"]), _ptr(meta["num_active"]),
                                _ptr(meta["sorted_weight"]), _stream(dev)), "moe_dispatch")
    return meta


def moe_combine(rows, topk_ids, topk_weights, num_experts, skip_padded_tokens=False, out=None):
    """Sum each token's k weighted route rows ([T*k, H] bf16) -> [T, H] bf16.

    Slots whose id lies outside [0, num_experts) are skipped, as the
    dispatch sorts them into the invalid bucket."""
    _require_gpu(rows, topk_ids, topk_weights)
    T, k = topk_ids.shape
    H = rows.shape[1]
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=rows.device)
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.bfloat16).contiguous()
    check(lib.qmoe_moe_combine(_ptr(rows), _ptr(ids), _ptr(wts), T, k, int(num_experts), H,
                               int(bool(skip_padded_tokens)), _ptr(out), out.stride(0),
                               _stream(rows.device)), "moe_combine")
    return out


# ---------------------------------------------------------------- fused decode MoE

DECODE_MAX_TOKENS = 64


def _f32c(t, shape, what):
    """float32 contiguous scales of `shape` (unit axes may differ)."""
    if t.numel() != math.prod(shape):
        raise ValueError(f"{what}: expected {tuple(shape)} float32 scales, got {tuple(t.shape)}")
    return t.float().reshape(shape).contiguous()


def moe_decode(hidden, w1, w2, w1_scale, w2_scale, shared_w1, shared_w1_scale, shared_w2, shared_w2_scale,
               shared_gate_weight, topk_weights, topk_ids, routed_scale=1.0, weight_blocks=None, out=None):
    """Fused decode MoE layer -- shared expert + routed experts -> bf16 [T, H]
    (`kernels/experimental/fused_moe_decode/fused_moe_decode_kernel.py:
    552-740` on one rank; the numerics are stated at `qmoe_moe_decode` in
    include/qmoe.h).

    Layouts (N-major, the layout the MoE methods keep): ``w1`` e4m3 [E, 2I, H]
    (gate rows then up rows), ``w2`` [E, H, I]; scales per channel ([E, 2I] /
    [E, H], trailing unit axes allowed) or, with ``weight_blocks=128``,
    128x128 tile scales ([E, 2I/128, H/128] / [E, H/128, I/128]). The shared
    expert's tensors drop the E axis ([2 I_s, H], [H, I_s]); ``I_s <= I``.
    ``shared_gate_weight``: [H] bf16 (any shape of H elements) or None for an
    ungated shared expert. ``routed_scale`` multiplies the routed experts
    only. 1..64 tokens."""
    _require_gpu(hidden, w1, w2, topk_ids, topk_weights)
    if tuple(topk_weights.shape) != tuple(topk_ids.shape):
        raise ValueError("moe_decode: inconsistent weight / routing shapes")
    ids = topk_ids.to(torch.int32).contiguous()
    f32w = topk_weights.dtype == torch.float32
    tw = topk_weights.contiguous() if f32w else topk_weights.to(torch.bfloat16).contiguous()
    return _moe_decode_call(hidden, w1, w2, w1_scale, w2_scale, shared_w1, shared_w1_scale, shared_w2,
                            shared_w2_scale, shared_gate_weight, tw, ids, routed_scale, weight_blocks, out, None)


def moe_decode_routed(hidden, router_logits, top_k, w1, w2, w1_scale, w2_scale, shared_w1, shared_w1_scale,
                      shared_w2, shared_w2_scale, shared_gate_weight, scoring_func="softmax", renormalize=True,
                      bias=None, routed_scaling_factor=1.0, num_expert_group=1, topk_group=1, routed_scale=1.0,
                      weight_blocks=None, out=None):
    """`moe_route` + `moe_decode` in one call: the op routes the tokens
    itself (for up to 8 tokens inside its first launch) with `moe_route`'s
    rule and arguments, then runs the fused decode layer. Returns (out bf16
    [T, H], topk_weights bf16 [T, k], topk_ids int32 [T, k]) -- the same
    values as the two calls. No counterpart in the reference, whose router
    runs before its decode kernel."""
    _require_gpu(hidden, router_logits, bias)
    if scoring_func not in _SCORING:
        raise NotImplementedError(f"FusedMoE does not support {scoring_func} scoring function for TPU.")
    x = router_logits.reshape(-1, router_logits.shape[-1])
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    T, E = x.shape
    if top_k > E:
        raise ValueError(f"topk k={top_k} exceeds the expert count {E}")
    if T != hidden.shape[0] or E != w1.shape[0]:
        raise ValueError("moe_decode_routed: router logits must be [T, E]")
    tw = torch.empty((T, top_k), dtype=torch.bfloat16, device=x.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    b = bias.float().contiguous() if bias is not None else None
    route = (x, b, _SCORING[scoring_func], renormalize, routed_scaling_factor, num_expert_group, topk_group)
    out = _moe_decode_call(hidden, w1, w2, w1_scale, w2_scale, shared_w1, shared_w1_scale, shared_w2,
                           shared_w2_scale, shared_gate_weight, tw, ids, routed_scale, weight_blocks, out, route)
    return out, tw, ids


def _moe_decode_call(hidden, w1, w2, w1_scale, w2_scale, shared_w1, shared_w1_scale, shared_w2, shared_w2_scale,
                     shared_gate_weight, tw, ids, routed_scale, weight_blocks, out, route):
    """Checks, the `qmoe_moe_decode_desc` and the call; `route` = (logits,
    bias, scoring, renormalize, rsf, num_group, topk_group) when the op
    routes (then `tw` / `ids` are its outputs)."""
    _require_gpu(hidden, w1, w2, ids, tw)
    T, H = hidden.shape
    E, N1, H1 = w1.shape
    I = N1 // 2
    Is = shared_w2.shape[1]
    k = ids.shape[1]
    if not 1 <= T <= DECODE_MAX_TOKENS:
        raise ValueError(f"moe_decode takes 1..{DECODE_MAX_TOKENS} tokens, got {T}")
    if H1 != H or tuple(w2.shape) != (E, H, I) or tuple(shared_w1.shape) != (2 * Is, H) or \
            tuple(shared_w2.shape) != (H, Is) or tuple(tw.shape) != (T, k):
        raise ValueError("moe_decode: inconsistent weight / routing shapes")
    for t, name in ((w1, "w1"), (w2, "w2"), (shared_w1, "shared_w1"), (shared_w2, "shared_w2")):
        if t.dtype != FP8 or not t.is_contiguous():
            raise ValueError(f"moe_decode: {name} must be a contiguous float8_e4m3fn tensor")
    tiles = bool(weight_blocks)
    if tiles and weight_blocks != 128:
        raise ValueError("moe_decode: weight_blocks must be None or 128")
    if tiles:
        s1 = _f32c(w1_scale, (E, N1 // 128, H // 128), "w1_scale")
        s2 = _f32c(w2_scale, (E, H // 128, I // 128), "w2_scale")
        ss1 = _f32c(shared_w1_scale, (2 * Is // 128, H // 128), "shared_w1_scale")
        ss2 = _f32c(shared_w2_scale, (H // 128, Is // 128), "shared_w2_scale")
    else:
        s1 = _f32c(w1_scale, (E, N1), "w1_scale")
        s2 = _f32c(w2_scale, (E, H), "w2_scale")
        ss1 = _f32c(shared_w1_scale, (2 * Is,), "shared_w1_scale")
        ss2 = _f32c(shared_w2_scale, (H,), "shared_w2_scale")
    x = hidden.to(torch.bfloat16).contiguous()
    if x.data_ptr() % 16:
        x = x.clone()  # the kernel reads 16-byte chunks
    gate = None
    if shared_gate_weight is not None:
        if shared_gate_weight.numel() != H:
            raise ValueError("moe_decode: shared_gate_weight must hold H values")
        gate = shared_gate_weight.reshape(H).to(torch.bfloat16).contiguous()
        if gate.data_ptr() % 16:
            gate = gate.clone()
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden.device)
    d = _capi.DecodeDesc()
    d.x = _ptr(x).value
    d.T, d.H, d.I, d.I_shared, d.E, d.topk = T, H, I, Is, E, k
    d.topk_ids = _ptr(ids).value
    d.topk_weights = _ptr(tw).value
    d.weights_f32 = int(tw.dtype == torch.float32)
    d.routed_scale = float(routed_scale)
    d.weight_blocks = 128 if tiles else 0
    d.w1, d.w2 = _ptr(w1).value, _ptr(w2).value
    d.w1_scale, d.w2_scale = _ptr(s1).value, _ptr(s2).value
    d.shared_w1, d.shared_w2 = _ptr(shared_w1).value, _ptr(shared_w2).value
    d.shared_w1_scale, d.shared_w2_scale = _ptr(ss1).value, _ptr(ss2).value
    d.shared_gate = _ptr(gate).value if gate is not None else None
    d.out = _ptr(out).value
    d.ldo = out.stride(0)
    if route is not None:
        lg, b, scoring, renorm, rsf, ng, tg = route
        d.router_logits = _ptr(lg).value
        d.logits_f32 = int(lg.dtype == torch.float32)
        d.scoring = scoring
        d.correction_bias = _ptr(b).value if b is not None else None
        d.renormalize = int(bool(renorm))
        d.routed_scaling_factor = float(rsf)
        d.num_group = int(ng or 1)
        d.topk_group = int(tg or 1)
    nbytes = ctypes.c_int64(0)
    check(lib.qmoe_moe_decode_workspace_size(ctypes.byref(d), ctypes.byref(nbytes)), "moe_decode (shape)")
    ws, ws_n = _workspace(hidden.device, nbytes.value)
    check(lib.qmoe_moe_decode(ctypes.byref(d), _ptr(ws), ws_n, _stream(hidden.device)), "moe_decode")
    return out


def stream_read(buf, workgroups=2048, sink=None):
    """Plain read of a device buffer (`qmoe_stream_read`): the HBM read floor
    the weight-streaming GEMMs are measured against. ``buf``'s byte size must
    be a multiple of 16; ``sink`` (int32 [workgroups]) is allocated when not
    given."""
    _require_gpu(buf)
    nbytes = buf.numel() * buf.element_size()
    if sink is None:
        sink = torch.empty(workgroups, dtype=torch.int32, device=buf.device)
    check(lib.qmoe_stream_read(_ptr(buf), nbytes, workgroups, _ptr(sink), _stream(buf.device)), "stream_read")
    return sink

