"""The C-ABI library loads (no GPU needed) and exports every function that
include/qmoe.h declares; host-side argument validation rejects bad input
before any launch."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "qmoe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*int(?:64_t)?\s+(qmoe_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_abi():
    names = _declared()
    assert "qmoe_gemm" in names and "qmoe_moe_dispatch" in names
    assert len(names) >= 7


def test_library_exports_every_declared_symbol():
    from qmoe import _capi

    for name in _declared():
        assert hasattr(_capi.lib, name), name
    assert set(_capi.EXPORTED) == set(_declared())
    assert _capi.lib.qmoe_abi_version() == _capi.ABI_VERSION


def test_gemm_desc_layout_matches_header_fields():
    from qmoe import _capi

    src = open(os.path.join(ROOT, "include", "qmoe.h")).read()
    body = src[src.index("typedef struct qmoe_gemm_desc"):src.index("} qmoe_gemm_desc;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split("{", 1)[1].split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.replace("*", " ").split()
        tail = decl.split()[-1]
        # "float act_p0, act_p1" declares two fields
        for part in decl.split(","):
            fields.append(part.replace("*", " ").split()[-1])
    assert [f for f, _ in _capi.GemmDesc._fields_] == fields


def test_invalid_descriptor_is_rejected_without_launch():
    from qmoe import _capi

    d = _capi.GemmDesc()
    d.kind = 99
    d.slots = 1
    n = ctypes.c_int64(0)
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 1
    assert _capi.lib.qmoe_gemm(ctypes.byref(d), None, 0, None) == 1
    # row quant: K not a multiple of 8
    assert _capi.lib.qmoe_row_quant(None, 0, 0, 1, 12, 0, 0, 0, None, 0, None, 0, None) == 1
    # router: topk > E
    assert _capi.lib.qmoe_moe_route(None, 0, 1, 4, 8, 0, None, 1, 1.0, 1, 1, None, 0, None, None) == 1
    # dispatch: too many experts
    assert _capi.lib.qmoe_moe_dispatch(None, None, 1, 1, 4096, 0, None, None, None, None, None, None,
                                       None, None) == 1


def test_product_path_has_no_cpu_fallback():
    import torch

    from qmoe import ops

    with pytest.raises(ValueError, match="device tensors"):
        ops.row_quant(torch.zeros(2, 16, dtype=torch.bfloat16))


def test_four_bit_descriptors_are_validated_on_the_host():
    """NVFP4 / INT4 descriptors: scale layout and group checks run in
    `qmoe_gemm_workspace_size` before any launch (pointer values are only
    checked for alignment, never dereferenced)."""
    from qmoe import _capi

    def desc(kind, K=1024, ldws=None, group=0, scale_ptr=0x1000):
        d = _capi.GemmDesc()
        d.kind, d.a, d.w, d.y, d.w_scale = kind, 0x1000, 0x1000, 0x1000, scale_ptr
        d.lda, d.ldw, d.ldy = K, K // 2, 256
        d.M, d.N, d.K, d.slots, d.max_rows = 4, 256, K, 1, 4
        d.ldws = ldws if ldws is not None else (K // 16 if kind == _capi.W4A16_NV else K // max(group, 1))
        d.wq_group = group
        return d

    n = ctypes.c_int64(0)
    ws = lambda d: _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n))  # noqa: E731
    assert ws(desc(_capi.W4A16_NV)) == 0
    assert ws(desc(_capi.W4A16_NV, ldws=32)) == 1            # fewer than K/16 scales per row
    assert ws(desc(_capi.W4A16_NV, scale_ptr=0x1002)) == 1   # bf16 pairs need 4-byte alignment
    for g in (32, 64, 128):
        assert ws(desc(_capi.W4A16_I4, group=g)) == 0
    assert ws(desc(_capi.W4A16_I4, group=48)) == 1           # groups of 32, 64 or 128 only
    assert ws(desc(_capi.W4A16_I4, group=0)) == 1
    assert ws(desc(_capi.W4A16_I4, K=1056, group=64)) == 1   # K not a multiple of the group
    assert ws(desc(_capi.W4A16_I4, group=32, scale_ptr=0x1001)) == 1


def test_dynamic_quant_kind_plans_on_the_host():
    """QMOE_W8A8_PC_DYN (bf16 rows quantized inside the call): one row runs
    the streaming kernel with the quantization inside; larger problems the
    plan of the per-channel GEMM after a separate quantization, whose codes
    and scales the workspace holds; grouped descriptors are refused."""
    from qmoe import _capi, ops

    for K, N in ((4096, 14336), (14336, 4096)):
        assert ops.plan_for_shape(_capi.W8A8_PC_DYN, 1, N, K)[4] == "stream_dyn"
    # one row: one K slice (few weight tiles would otherwise split K); rows
    # under 1024 columns quantize in a launch of their own
    for K, N in ((7168, 1536), (7168, 576)):
        assert ops.plan_for_shape(_capi.W8A8_PC_DYN, 1, N, K)[4:] == ("stream_dyn", 16, 1)
        assert ops.plan_for_shape(_capi.W8A8_PC, 1, N, K)[6] > 1
    assert ops.plan_for_shape(_capi.W8A8_PC_DYN, 1, 32768, 512)[4] == "stream"
    for K, N in ((4096, 14336), (14336, 4096)):
        for M in (8, 64, 4096):
            assert ops.plan_for_shape(_capi.W8A8_PC_DYN, M, N, K)[4:] == ops.plan_for_shape(_capi.W8A8_PC, M, N, K)[4:]
    d = _capi.GemmDesc()
    d.kind, d.a, d.w, d.y, d.w_scale = _capi.W8A8_PC_DYN, 1 << 24, 1 << 24, 1 << 24, 1 << 24
    d.lda, d.ldw, d.ldy, d.ldws = 4096, 4096, 1024, 1
    d.M, d.N, d.K, d.slots, d.max_rows = 64, 1024, 4096, 1, 64
    n = ctypes.c_int64(0)
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value >= 64 * 4096 + 64 * 4  # the codes and scales of the separate quantization
    d.M = d.max_rows = 1
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value >= 4  # the row scale
    d.group_offs, d.slots = 1 << 24, 2
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 1


def test_weight_code_formats_are_validated_on_the_host():
    """wfmt 0 e4m3, 1 int8, 2 e5m2 for the per-channel, grouped-matmul and
    in-call-quantization W8A8 kinds; any other value, and a nonzero wfmt on
    the other kinds, is refused before a launch. e5m2 plans the same kernels
    as e4m3 (the 1-byte tiles and the streaming kernel take both formats)."""
    from qmoe import _capi, ops

    for kind in (_capi.W8A8_PC, _capi.W8A8_GMM, _capi.W8A8_PC_DYN):
        for M in (1, 64, 4096):
            e4 = ops.plan_for_shape(kind, M, 4096, 4096, wfmt=0)
            assert ops.plan_for_shape(kind, M, 4096, 4096, wfmt=2)[2:] == e4[2:]
    d = _capi.GemmDesc()
    d.kind, d.a, d.w, d.y, d.w_scale, d.a_scale = _capi.W8A8_PC, 1 << 24, 1 << 24, 1 << 24, 1 << 24, 1 << 24
    d.lda, d.ldw, d.ldy, d.ldws, d.lds_a = 4096, 4096, 1024, 1, 1
    d.M, d.N, d.K, d.slots, d.max_rows = 64, 1024, 4096, 1, 64
    n = ctypes.c_int64(0)
    for wfmt, rc in ((0, 0), (1, 0), (2, 0), (3, 1), (-1, 1)):
        d.wfmt = wfmt
        assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == rc, wfmt
    d.kind, d.wfmt = _capi.W8A16_PC, 2
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 1


def test_under_filled_prefill_plans_on_the_host():
    """Prefill problems that one tile per workgroup would leave under-filled:
    dense bf16-activation problems under 256 tiles of 128 x 128 split K into
    about 512 workgroups (at most 8 slices of at least 8 stages), with the
    f32 slices sized in the workspace; per-channel 1-byte problems of at
    most 1024 channels over 256 tokens take 128-row weight tiles of 64 or
    128 tokens (the larger once the smaller would make over 256 tiles)."""
    from qmoe import _capi, ops

    # DeepSeek-V3's bf16 router gate (K 7168, N 256)
    for M, ks in ((65, 8), (4096, 8), (8192, 4), (16384, 1)):
        assert ops.plan_for_shape(_capi.W16A16, M, 256, 7168)[4:] == ("tiled_generic", 128, ks), M
    assert ops.plan_for_shape(_capi.W8A16_PC, 4096, 256, 7168)[4:] == ("tiled_generic", 128, 8)
    # a short K keeps one slice; a fused activation never splits
    assert ops.plan_for_shape(_capi.W16A16, 1000, 256, 512)[6] == 1
    assert ops.plan_for_shape(_capi.W16A16, 4096, 512, 7168, activation="silu")[6] == 1
    d = _capi.GemmDesc()
    d.kind, d.a, d.w, d.y = _capi.W16A16, 1 << 24, 1 << 24, 1 << 24
    d.lda, d.ldw, d.ldy = 7168, 2 * 7168, 256
    d.M, d.N, d.K, d.slots, d.max_rows = 4096, 256, 7168, 1, 4096
    n = ctypes.c_int64(0)
    assert _capi.lib.qmoe_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == 8 * 4096 * 256 * 4
    # DeepSeek-V3's kv_a projection (576 channels) and a ragged 1000-channel problem
    for wf in (0, 1):
        assert ops.plan_for_shape(_capi.W8A8_PC, 2000, 576, 7168, wfmt=wf)[4:] == ("tiled_1b_n128", 64, 1)
        assert ops.plan_for_shape(_capi.W8A8_PC, 4096, 576, 7168, wfmt=wf)[4:] == ("tiled_1b_n128", 128, 1)
        assert ops.plan_for_shape(_capi.W8A8_PC, 4096, 1000, 4096, wfmt=wf)[4:] == ("tiled_1b_n128", 128, 1)
