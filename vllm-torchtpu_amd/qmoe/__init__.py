"""qmoe: MI355X (gfx950) quantized GEMM and fused MoE behind the vllm-torchtpu
quant-method / fused-MoE operator surface.

Layout of the package:
  _capi.py   ctypes binding of libqmoe.so (C ABI in include/qmoe.h)
  ops.py     torch-facing wrappers (device tensors only)
  layers/    mirrors of the reference plugin's adapter entry points
"""

__all__ = ["ops"]
