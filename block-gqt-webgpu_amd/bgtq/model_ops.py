"""The model step's kernel protocol: ModelOps / Commands of src/model/ops.ts.

ModelOps.create(device).commands() records dispatch(name, parameters,
buffers, x, y) calls and submit() runs them in order on the device's stream
and waits, as the reference's Commands does (src/model/ops.ts:21-31). The
names on the attention path are served by libbgtq.so (bgtq_model_submit):
append, encode_k, dot, compressed_dot, softmax and weighted, with the
reference's parameter arrays, binding orders and buffer layouts (as
src/model/decoder.ts:46-56 dispatches them). The model's other kernels
(embedding, matmul, norm, element, rope) raise UnsupportedError.

A buffer is a torch tensor on the GPU (device memory only: torch is the
allocator here, the arithmetic runs in the library's kernels), or, for the
config and table slots of encode_k and compressed_dot, the head's calibration
tables (a Calibration head's .config / .table, or a Tables object).
"""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import RangeError, check, lib

# Largest workgroup count per dimension a dispatch may name (the reference
# checks device.limits.maxComputeWorkgroupsPerDimension, src/model/ops.ts:26).
MAX_WORKGROUPS_PER_DIMENSION = 0x7FFFFFFF

ATTENTION_PATH = ("append", "encode_k", "dot", "compressed_dot", "softmax", "weighted")


def _binding(b) -> _lib.Binding:
    if b is None:
        return _lib.Binding(None, 0, None)
    handle = getattr(b, "handle", None)
    if handle is not None and hasattr(b, "info"):  # calibration Tables
        return _lib.Binding(None, 0, handle)
    if not b.is_contiguous():
        raise RangeError("Model buffers must be contiguous")
    return _lib.Binding(ctypes.c_void_p(b.data_ptr()), b.numel() * b.element_size(), None)


class ModelOps:
    def __init__(self, device):
        self.device = device

    @classmethod
    def create(cls, device) -> "ModelOps":
        return cls(device)

    def commands(self) -> "Commands":
        return Commands(self)


class Commands:
    def __init__(self, ops: ModelOps):
        self.ops = ops
        self._dispatches: list[tuple[str, list[int], list, int, int]] = []

    def dispatch(self, name: str, parameters, buffers, x: int, y: int = 1) -> None:
        if x > MAX_WORKGROUPS_PER_DIMENSION or y > MAX_WORKGROUPS_PER_DIMENSION:
            raise RangeError("Model dispatch limit")
        params = [int(v) & 0xFFFFFFFF for v in list(parameters)[:8]]
        self._dispatches.append((name, params + [0] * (8 - len(params)), list(buffers), int(x), int(y)))

    def submit(self) -> None:
        """Queue every recorded dispatch in order, then wait for the device.
        A dispatch that fails its checks raises before anything is queued."""
        n = len(self._dispatches)
        arr = (_lib.ModelDispatch * max(1, n))()
        keep = []
        for i, (name, params, buffers, x, y) in enumerate(self._dispatches):
            binds = (_lib.Binding * max(1, len(buffers)))(*[_binding(b) for b in buffers])
            keep.append(binds)
            encoded = name.encode()
            keep.append(encoded)
            arr[i] = _lib.ModelDispatch(encoded, (ctypes.c_uint32 * 8)(*params),
                                        ctypes.cast(binds, ctypes.POINTER(_lib.Binding)), len(buffers), x, y)
        self._dispatches = []
        check(lib().bgtq_model_submit(self.ops.device.handle, arr, n))
        self.ops.device.synchronize()
