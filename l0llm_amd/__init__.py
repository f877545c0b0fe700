"""l0llm_amd: MI355X (gfx950) decoder matmul and decode-attention path of l0llm.

The compute lives in libl0hip.so (hand-written HIP for gfx950, C ABI in include/l0hip.h).
This package is the Python host side over that ABI, mirroring the reference's operator
interface (LlmKernelSuite, LlmMatrix, LlmModel). Importing it loads the library; a missing
library is an ImportError, never a CPU fallback."""
from ._lib import (BF16, F16, F32, I8PC, PRECISION_AUTO, PRECISION_BFLOAT16, PRECISION_FLOAT16,
                   PRECISION_FLOAT32, PRECISION_INT8, DeviceError, InvalidArgumentError, InvalidDataError,
                   InvalidOperationError, L0hError, UnsupportedError, declared_functions, lib)
from .api import (Buffer, Device, HfConfig, LlmKernelSuite, LlmMatrix, LlmModel, RopeScaling, SafetensorsCheckpoint,
                  fits_in_half, quantize_i8pc, rope_frequencies, runtime_is_available, transpose)

__all__ = [
    "BF16", "F16", "F32", "I8PC", "PRECISION_AUTO", "PRECISION_BFLOAT16", "PRECISION_FLOAT16", "PRECISION_FLOAT32",
    "PRECISION_INT8", "Buffer", "Device", "DeviceError", "HfConfig", "InvalidArgumentError", "InvalidDataError",
    "InvalidOperationError", "L0hError", "LlmKernelSuite", "LlmMatrix", "LlmModel", "RopeScaling",
    "SafetensorsCheckpoint", "UnsupportedError", "declared_functions", "fits_in_half", "lib", "quantize_i8pc", "rope_frequencies",
    "runtime_is_available", "transpose",
]
