"""Quant-config registry (the reference's
`layers/adapter/quantization/__init__.py:51-101`, `get_tpu_quantization_config`):
maps a checkpoint's ``quantization`` method name to the config class."""

from qmoe.layers.quantization.compressed_tensors import (CompressedTensorsConfig, CompressedTensorsW4A16MoEMethod,
                                                        CompressedTensorsW4ANMxfp4MoEMethod)
from qmoe.layers.quantization.fp8 import Fp8Config, Fp8LinearMethod, Fp8MoEMethod
from qmoe.layers.quantization.mxfp4 import Mxfp4Config, Mxfp4LinearMethod, Mxfp4MoEMethod
from qmoe.layers.quantization.nvfp4 import Nvfp4Config, Nvfp4LinearMethod, Nvfp4MoEMethod
from qmoe.layers.quantization.unquantized import UnquantizedFusedMoEMethod, UnquantizedLinearMethod

_CONFIGS = {
    "fp8": Fp8Config,
    "mxfp4": Mxfp4Config,
    "modelopt_fp4": Nvfp4Config,
    "compressed-tensors": CompressedTensorsConfig,
}


def get_quantization_config(method: str):
    """Config class for a checkpoint quantization method name."""
    try:
        return _CONFIGS[method]
    except KeyError:
        raise ValueError(
            f"{method} quantization is not supported by qmoe (supported: {', '.join(sorted(_CONFIGS))})"
        ) from None


__all__ = [
    "CompressedTensorsConfig", "CompressedTensorsW4A16MoEMethod", "CompressedTensorsW4ANMxfp4MoEMethod", "Fp8Config", "Fp8LinearMethod", "Fp8MoEMethod", "Mxfp4Config", "Mxfp4LinearMethod",
    "Mxfp4MoEMethod", "Nvfp4Config", "Nvfp4LinearMethod", "Nvfp4MoEMethod", "UnquantizedFusedMoEMethod", "UnquantizedLinearMethod",
    "get_quantization_config",
]
