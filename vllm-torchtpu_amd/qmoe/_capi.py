"""ctypes binding of libqmoe.so (the C ABI declared in include/qmoe.h).

The library is required: if it is missing or does not load, importing this
module raises, so no call can silently run anything but the HIP kernels.

torch is imported before the library is loaded: the PyTorch wheel carries
its own HIP runtime (``torch/lib/libamdhip64.so``, the same soname as
ROCm's), and libqmoe.so must bind to that one. Loaded first, it would bind
to ROCm's copy and torch would then load its own: two runtimes in one
process, whose streams and allocations the other does not know (kernel
launches on torch's streams then fail).
"""

import ctypes
import os

import torch  # noqa: F401  (its HIP runtime first; see above)

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqmoe.so")

ABI_VERSION = 8

QMOE_OK = 0
STATUS_TEXT = {
    1: "invalid argument (shape, layout or unsupported combination)",
    2: "workspace too small",
    3: "kernel launch failed",
    4: "the problem's split-K partial sums exceed the static scratch of qmoe_gemm_static (64 MiB)",
}

# GEMM kinds / activations (include/qmoe.h)
(W8A8_PC, W8A8_BLK, W8A16_PC, W4A16_MX, W16A16, W4A16_NV, W4A16_I4, W8A8_GMM, W8A16_BLK, W4A4_MX,
 W8A8_PC_DYN) = range(11)
ACT_NONE, ACT_SILU, ACT_SWIGLUOAI, ACT_GELU_TANH, ACT_SILU_CLAMP, ACT_SITU = range(6)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class GemmDesc(ctypes.Structure):
    """Mirror of `qmoe_gemm_desc` (field order and types must match)."""

    _fields_ = [
        ("kind", _i32),
        ("wfmt", _i32),
        ("a", _vp),
        ("lda", _i64),
        ("a_scale", _vp),
        ("lds_a", _i64),
        ("a_rows", _vp),
        ("w", _vp),
        ("ldw", _i64),
        ("w_gstride", _i64),
        ("w_scale", _vp),
        ("ldws", _i64),
        ("ws_gstride", _i64),
        ("ws_bn", _i32),
        ("bias", _vp),
        ("bias_gstride", _i64),
        ("group_offs", _vp),
        ("active", _vp),
        ("num_active", _vp),
        ("slots", _i32),
        ("max_rows", _i32),
        ("M", _i32),
        ("N", _i32),
        ("K", _i32),
        ("act", _i32),
        ("act_p0", _f32),
        ("act_p1", _f32),
        ("row_weight", _vp),
        ("y", _vp),
        ("ldy", _i64),
        ("y_rows", _vp),
        ("wq_group", _i32),
    ]


class DecodeDesc(ctypes.Structure):
    """Mirror of `qmoe_moe_decode_desc` (field order and types must match)."""

    _fields_ = [
        ("x", _vp),
        ("T", _i64),
        ("H", _i64),
        ("I", _i64),
        ("I_shared", _i64),
        ("E", _i32),
        ("topk", _i32),
        ("topk_ids", _vp),
        ("topk_weights", _vp),
        ("weights_f32", _i32),
        ("routed_scale", _f32),
        ("weight_blocks", _i32),
        ("w1", _vp),
        ("w2", _vp),
        ("w1_scale", _vp),
        ("w2_scale", _vp),
        ("shared_w1", _vp),
        ("shared_w2", _vp),
        ("shared_w1_scale", _vp),
        ("shared_w2_scale", _vp),
        ("shared_gate", _vp),
        ("out", _vp),
        ("ldo", _i64),
        ("router_logits", _vp),
        ("logits_f32", _i32),
        ("scoring", _i32),
        ("correction_bias", _vp),
        ("renormalize", _i32),
        ("routed_scaling_factor", _f32),
        ("num_group", _i32),
        ("topk_group", _i32),
    ]


def _load():
    if not os.path.exists(_LIB_PATH):
        raise ImportError(
            f"qmoe: {_LIB_PATH} not found; build it with "
            "`python vllm-torchtpu_amd/qmoe/build.py` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(_LIB_PATH)
    lib.qmoe_abi_version.restype = ctypes.c_int
    lib.qmoe_abi_version.argtypes = []
    lib.qmoe_row_quant.restype = ctypes.c_int
    lib.qmoe_row_quant.argtypes = [_vp, _i64, ctypes.c_int, _i64, _i64, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, _vp, _i64, _vp, _i64, _vp]
    lib.qmoe_mx_quant.restype = ctypes.c_int
    lib.qmoe_mx_quant.argtypes = [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp]
    lib.qmoe_gemm_workspace_size.restype = ctypes.c_int
    lib.qmoe_gemm_workspace_size.argtypes = [ctypes.POINTER(GemmDesc), ctypes.POINTER(_i64)]
    lib.qmoe_gemm_plan.restype = ctypes.c_int
    lib.qmoe_gemm_plan.argtypes = [ctypes.POINTER(GemmDesc), ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                                   ctypes.POINTER(_i32)]
    lib.qmoe_gemm_static.restype = ctypes.c_int
    lib.qmoe_gemm_static.argtypes = [ctypes.POINTER(GemmDesc), _vp]
    lib.qmoe_gemm_static_scratch_bytes.restype = _i64
    lib.qmoe_gemm_static_scratch_bytes.argtypes = []
    lib.qmoe_gemm.restype = ctypes.c_int
    lib.qmoe_gemm.argtypes = [ctypes.POINTER(GemmDesc), _vp, _i64, _vp]
    lib.qmoe_moe_route.restype = ctypes.c_int
    lib.qmoe_moe_route.argtypes = [_vp, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   _vp, ctypes.c_int, _f32, ctypes.c_int, ctypes.c_int, _vp,
                                   ctypes.c_int, _vp, _vp]
    lib.qmoe_moe_dispatch.restype = ctypes.c_int
    lib.qmoe_moe_dispatch.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.qmoe_moe_route_dispatch.restype = ctypes.c_int
    lib.qmoe_moe_route_dispatch.argtypes = [_vp, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            _vp, ctypes.c_int, _f32, ctypes.c_int, ctypes.c_int, _vp, _vp,
                                            ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.qmoe_moe_route_hash.restype = ctypes.c_int
    lib.qmoe_moe_route_hash.argtypes = [_vp, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp,
                                        _i64, _vp, ctypes.c_int, ctypes.c_int, _f32, _vp, _vp, _vp]
    lib.qmoe_moe_combine.restype = ctypes.c_int
    lib.qmoe_moe_combine.argtypes = [_vp, _vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _i64, ctypes.c_int, _vp,
                                     _i64, _vp]
    lib.qmoe_moe_decode_workspace_size.restype = ctypes.c_int
    lib.qmoe_moe_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeDesc), ctypes.POINTER(_i64)]
    lib.qmoe_moe_decode.restype = ctypes.c_int
    lib.qmoe_moe_decode.argtypes = [ctypes.POINTER(DecodeDesc), _vp, _i64, _vp]
    lib.qmoe_stream_read.restype = ctypes.c_int
    lib.qmoe_stream_read.argtypes = [_vp, _i64, _i32, _vp, _vp]
    v = lib.qmoe_abi_version()
    if v != ABI_VERSION:
        raise ImportError(f"qmoe: libqmoe.so ABI {v} != expected {ABI_VERSION}; rebuild it")
    return lib


lib = _load()

EXPORTED = (
    "qmoe_abi_version",
    "qmoe_stream_read",
    "qmoe_row_quant",
    "qmoe_mx_quant",
    "qmoe_gemm_workspace_size",
    "qmoe_gemm_plan",
    "qmoe_gemm_static",
    "qmoe_gemm_static_scratch_bytes",
    "qmoe_gemm",
    "qmoe_moe_route",
    "qmoe_moe_dispatch",
    "qmoe_moe_route_dispatch",
    "qmoe_moe_route_hash",
    "qmoe_moe_combine",
    "qmoe_moe_decode_workspace_size",
    "qmoe_moe_decode",
)


def check(status: int, what: str) -> None:
    if status != QMOE_OK:
        raise RuntimeError(f"qmoe: {what} failed: {STATUS_TEXT.get(status, status)}")
