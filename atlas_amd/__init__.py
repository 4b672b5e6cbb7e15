"""atlas_amd -- MI355X (gfx950) fused per-layer elementwise / normalisation ops.

The compute lives in libatlas_hip_ops.so (hand-written HIP, C ABI in
include/atlas_hip_ops.h).  Importing this package does not touch the GPU;
constructing a HipRuntime / NeuralOps loads the library and fails loudly if
it was not built or no device is present.
"""
from ._lib import (ATLAS_ERR_COMMAND_FAILED, ATLAS_ERR_INVALID_INPUT, ATLAS_ERR_NO_DEVICE, ATLAS_OK,
                   ATLAS_REDUCTION_AUTO, ATLAS_REDUCTION_SEQUENTIAL, ATLAS_REDUCTION_WIDE, LIB_PATH,
                   DispatchTiming, load)
from .runtime import (DeviceBuffer, HipRuntime, NeuralOps, OperatorError, rope_tables_gemma4,
                      rope_tables_llama)

__all__ = [
    "ATLAS_OK", "ATLAS_ERR_NO_DEVICE", "ATLAS_ERR_INVALID_INPUT", "ATLAS_ERR_COMMAND_FAILED",
    "ATLAS_REDUCTION_AUTO", "ATLAS_REDUCTION_SEQUENTIAL", "ATLAS_REDUCTION_WIDE", "LIB_PATH", "DispatchTiming", "load",
    "DeviceBuffer", "HipRuntime", "NeuralOps", "OperatorError", "rope_tables_gemma4", "rope_tables_llama",
]
