"""Hot-path flags, read from the environment (names and meanings follow the
reference plugin's `envs.py`, `:43-97, 503-535, 725-750`).

Values are read when accessed (``envs.NAME``), so tests can monkeypatch the
environment; the quant methods read them at construction / load time, never
inside a forward call.
"""

import os


def _bool(name, default=False):
    v = os.getenv(name)
    if v is None:
        return default
    return v.strip().lower() in ("1", "true", "yes", "on")


def _opt_int(name):
    v = os.getenv(name)
    return int(v) if v not in (None, "") else None


def _nonneg_int(name, default):
    v = os.getenv(name)
    if v in (None, ""):
        return default
    iv = int(v)
    if iv < 0:
        raise ValueError(f"{name} must be >= 0, got {iv}")
    return iv


_READERS = {
    # dense linears: blockwise runtime kernel + its K block (both or neither)
    "ENABLE_QUANTIZED_MATMUL_KERNEL": lambda: _bool("ENABLE_QUANTIZED_MATMUL_KERNEL"),
    "REQUANTIZE_BLOCK_SIZE": lambda: _opt_int("REQUANTIZE_BLOCK_SIZE"),
    # dense linears: runtime weight dtype ("float8_e4m3fn" or "int8")
    "REQUANTIZE_WEIGHT_DTYPE": lambda: os.getenv("REQUANTIZE_WEIGHT_DTYPE", "float8_e4m3fn"),
    # FP8 dense linears keep bf16 activations for steps of at most this many rows
    "TPU_FP8_LINEAR_W8A16_MAX_ROWS": lambda: _nonneg_int("TPU_FP8_LINEAR_W8A16_MAX_ROWS", 0),
    # MoE: weight block size to requantize checkpoint experts to (NVFP4, INT4)
    "MOE_REQUANTIZE_BLOCK_SIZE": lambda: _opt_int("MOE_REQUANTIZE_BLOCK_SIZE"),
    # MoE: weight dtype to requantize packed-int4 experts to (e.g. "fp4")
    "MOE_REQUANTIZE_WEIGHT_DTYPE": lambda: os.getenv("MOE_REQUANTIZE_WEIGHT_DTYPE"),
    # MoE: routes with a zero routing weight are padding and skipped
    "TPU_MOE_SKIP_PADDED_TOKENS": lambda: _bool("TPU_MOE_SKIP_PADDED_TOKENS"),
    # MoE: steps of at most this many tokens (0: off) with per-channel FP8
    # experts, silu and no biases take the dense-expert decode semantics
    "TPU_MOE_DENSE_EXPERT_THRESHOLD": lambda: _nonneg_int("TPU_MOE_DENSE_EXPERT_THRESHOLD", 0),
    # MoE decode: serve armed layers' decode steps with the fused decode op
    # (shared + routed experts), up to MAX_TOKENS tokens per step
    "FUSED_MOE_DECODE_KERNEL": lambda: _bool("FUSED_MOE_DECODE_KERNEL"),
    "FUSED_MOE_DECODE_KERNEL_MAX_TOKENS": lambda: int(os.getenv("FUSED_MOE_DECODE_KERNEL_MAX_TOKENS", "256")),
    # this build only: the most tokens an armed layer's step serves with the
    # fused decode op before the GMM path (faster above it on MI355X; see
    # `qmoe/layers/fused_moe_decode.py`), whatever the cap above allows (0:
    # the cap alone)
    "QMOE_DECODE_OP_MAX_TOKENS": lambda: _nonneg_int("QMOE_DECODE_OP_MAX_TOKENS", 16),
    # this build only (no reference counterpart): 128x128-block FP8 checkpoints
    # keep their tiles at run time with per-(token, 128) e4m3 activations
    # (the blockwise W8A8 recipe of BASELINE configs 2 and 4) instead of the
    # reference's requantization (per channel for the MoE and without
    # REQUANTIZE_BLOCK_SIZE, per (row, block) otherwise)
    "QMOE_FP8_NATIVE_BLOCKS": lambda: _bool("QMOE_FP8_NATIVE_BLOCKS"),
    # this build only (no reference counterpart): dense MXFP4 linears quantize
    # their activations to MXFP4 too (W4A4, e2m1 + e8m0 per 32 columns) and
    # run the MX MFMA kernel; off: bf16 activations (W4A16) as the reference
    "QMOE_MXFP4_MX_ACTIVATIONS": lambda: _bool("QMOE_MXFP4_MX_ACTIVATIONS"),
}


def __getattr__(name):
    if name in _READERS:
        return _READERS[name]()
    raise AttributeError(name)


def __dir__():
    return list(_READERS)
