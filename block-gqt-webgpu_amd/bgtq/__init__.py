"""Block-GTQ on MI355X: the reference's runtime/attention classes over libbgtq.so.

Same names and semantics as the reference's TypeScript runtime
(src/runtime/*, src/attention/*, src/webgpu/layout.ts); every computation runs
in the HIP kernels of libbgtq.so. Importing requires the built library.
"""
from ._lib import (DeviceError, RangeError, StateError, UnsupportedError, LIB_PATH, lib)
from .layout import BlockGTQParameters, tables, validate_layout
from .runtime import (CompressedKeys, Device, FP16Keys, PackedKeys, Tables, Timestamps, Values, append_count)
from .attention import AttentionEngine, AttentionSession, OptimizedAttention
from .calibration import Calibration
from .model_ops import Commands, ModelOps

lib()  # fail loudly at import when the native library is missing

__all__ = ["BlockGTQParameters", "tables", "validate_layout", "Device", "Tables", "Timestamps", "FP16Keys", "PackedKeys",
           "CompressedKeys", "Values", "append_count", "AttentionEngine", "AttentionSession",
           "OptimizedAttention", "Calibration", "ModelOps", "Commands", "RangeError", "StateError", "DeviceError", "UnsupportedError", "LIB_PATH"]
