"""Cache stores: FP16Keys, PackedKeys, CompressedKeys, Values.

Mirrors src/runtime/keys.ts, packed-keys.ts, compressed-keys.ts and
values.ts: same constructors (create(device, parameters, capacity)), methods,
validation order and messages, allocation ledger with roles. The device work
runs in libbgtq.so on gfx950; the reference's async append() completes before
returning here (its Promise resolves after onSubmittedWorkDone).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import RangeError, StateError, check, lib, ptr
from .layout import BlockGTQParameters, tables


class Device:
    """A HIP device and the stream all work is ordered on (GPUDevice + queue)."""

    def __init__(self, index: int = 0):
        h = ctypes.c_void_p()
        check(lib().bgtq_context_create(index, ctypes.byref(h)))
        self.handle = h
        self.index = index

    def synchronize(self):
        check(lib().bgtq_context_synchronize(self.handle))

    def set_stream(self, stream_ptr: int | None):
        check(lib().bgtq_context_set_stream(self.handle, stream_ptr))

    def destroy(self):
        if self.handle:
            lib().bgtq_context_destroy(self.handle)
            self.handle = None


class Timestamps:
    """A timestamp query set (device.createQuerySet({type: "timestamp", count}),
    benchmarks/timing.ts:13-20): write(i) marks the time the work queued
    before it on the device's stream completed; resolve() gives nanoseconds."""

    def __init__(self, device: Device, count: int):
        h = ctypes.c_void_p()
        check(lib().bgtq_timestamps_create(device.handle, int(count), ctypes.byref(h)))
        self.handle, self.count = h, int(count)

    def write(self, index: int) -> None:
        check(lib().bgtq_timestamps_write(self.handle, int(index)))

    def resolve(self, first: int = 0, count: int | None = None) -> np.ndarray:
        n = self.count - first if count is None else int(count)
        out = np.zeros(n, np.uint64)
        check(lib().bgtq_timestamps_resolve(self.handle, int(first), n,
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))))
        return out

    def destroy(self) -> None:
        if self.handle:
            lib().bgtq_timestamps_destroy(self.handle)
            self.handle = None


class Tables:
    """Validated calibration tables resident on the device (tables(p))."""

    def __init__(self, device: Device, p: BlockGTQParameters | None = None, *, integer=None, floating=None):
        if p is not None:
            integer, floating = tables(p)
        integer = np.ascontiguousarray(integer, dtype=np.uint32)
        floating = np.ascontiguousarray(floating, dtype=np.float32)
        h = ctypes.c_void_p()
        check(lib().bgtq_tables_create(device.handle, ptr(integer), integer.size, ptr(floating), floating.size,
                                       ctypes.byref(h)))
        self.handle = h
        self.device = device
        info = _lib.TablesInfo()
        check(lib().bgtq_tables_info_get(h, ctypes.byref(info)))
        self.info = {k: getattr(info, k) for k, _ in info._fields_}

    def destroy(self):
        if self.handle:
            lib().bgtq_tables_destroy(self.handle)
            self.handle = None


def append_count(values, dim: int, length: int, capacity: int) -> int:
    """appendCount (src/runtime/keys.ts:11-15)."""
    v = np.asarray(values, dtype=np.uint16)
    if not v.size or v.size % dim:
        raise RangeError("K append must contain whole nonempty rows")
    if np.any((v & 0x7C00) == 0x7C00):
        raise RangeError("Finite FP16 K required")
    count = v.size // dim
    if length + count > capacity:
        raise RangeError("K capacity exceeded")
    return count


class _Keys:
    kind = ""

    def __init__(self, device: Device, handle):
        self.device = device
        self.handle = handle

    @property
    def dim(self) -> int:
        return lib().bgtq_keys_dim(self.handle)

    @property
    def capacity(self) -> int:
        return lib().bgtq_keys_capacity(self.handle)

    @property
    def length(self) -> int:
        return lib().bgtq_keys_length(self.handle)

    @property
    def allocations(self):
        return _lib.allocations(lib().bgtq_keys_allocations, self.handle)

    def append(self, values) -> None:
        """FP16 bit patterns of whole rows (Uint16Array in the reference)."""
        v = np.ascontiguousarray(np.asarray(values).reshape(-1))
        if v.dtype == np.float16:
            v = v.view(np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        check(lib().bgtq_keys_append(self.handle, ptr(v), v.size))

    def destroy(self) -> None:
        if self.handle:
            lib().bgtq_keys_destroy(self.handle)
            self.handle = None


class FP16Keys(_Keys):
    """src/runtime/keys.ts:16-27."""
    kind = "fp16"

    def __init__(self, device: Device, dim: int, capacity: int):
        h = ctypes.c_void_p()
        check(lib().bgtq_fp16_keys_create(device.handle, int(dim), int(capacity), ctypes.byref(h)))
        super().__init__(device, h)

    def read(self) -> np.ndarray:
        out = np.zeros(self.capacity * self.dim, np.uint16)
        check(lib().bgtq_keys_read_fp16(self.handle, ptr(out), out.size))
        return out


class PackedKeys(_Keys):
    """src/runtime/packed-keys.ts:7-52 (phase 4: packed rows, no decode scratch)."""
    kind = "block-gtq"
    _create = "bgtq_packed_keys_create"

    def __init__(self, device: Device, tables_: Tables, capacity: int, parameters=None):
        h = ctypes.c_void_p()
        check(getattr(lib(), self._create)(tables_.handle, int(capacity), ctypes.byref(h)))
        super().__init__(device, h)
        self.tables = tables_
        self.parameters = parameters
        self.row_bytes = tables_.info["row_bytes"]
        self.norm_stride = tables_.info["norm_stride"]

    @classmethod
    def create(cls, device: Device, p: BlockGTQParameters, capacity: int):
        if not isinstance(capacity, (int, np.integer)) or capacity < 1:
            raise RangeError("Invalid capacity")
        return cls(device, Tables(device, p), int(capacity), parameters=p)

    def ready(self) -> None:
        check(lib().bgtq_keys_ready(self.handle))

    def read(self):
        """(packed [capacity*rowBytes] uint8, norms [capacity*normStride] uint16)."""
        packed = np.zeros(self.capacity * self.row_bytes, np.uint8)
        norms = np.zeros(self.capacity * self.norm_stride, np.uint16)
        check(lib().bgtq_keys_read_packed(self.handle, ptr(packed), packed.size, ptr(norms), norms.size))
        return packed, norms

    def destroy(self) -> None:
        super().destroy()
        if getattr(self, "parameters", None) is not None and self.tables is not None:
            self.tables.destroy()
            self.tables = None


class CompressedKeys(PackedKeys):
    """src/runtime/compressed-keys.ts:5-59 (phase 3: materialises FP32 K for attention)."""
    _create = "bgtq_compressed_keys_create"

    def prepare(self) -> np.ndarray:
        """Materialise FP32 K rows [length, dim] (KeyView{format:"f32"})."""
        out = np.zeros((self.length, self.dim), np.float32)
        check(lib().bgtq_keys_prepare(self.handle, ptr(out), out.size))
        return out


class Values:
    """src/runtime/values.ts:3-16. dtype "f32" (synthetic path) or "f16" (model path)."""

    def __init__(self, device: Device, dim: int, capacity: int, dtype: str = "f32"):
        if not isinstance(dim, (int, np.integer)) or not isinstance(capacity, (int, np.integer)):
            raise RangeError("Invalid V dimensions")
        h = ctypes.c_void_p()
        code = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16}.get(dtype)
        if code is None:
            raise RangeError("Invalid V dimensions")
        check(lib().bgtq_values_create(device.handle, int(dim), int(capacity), code, ctypes.byref(h)))
        self.device, self.handle, self.dim, self.capacity, self.dtype = device, h, int(dim), int(capacity), dtype

    @property
    def length(self) -> int:
        return lib().bgtq_values_length(self.handle)

    @property
    def allocations(self):
        return _lib.allocations(lib().bgtq_values_allocations, self.handle)

    def append(self, values) -> None:
        v = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
        check(lib().bgtq_values_append(self.handle, ptr(v), v.size))

    def destroy(self) -> None:
        if self.handle:
            lib().bgtq_values_destroy(self.handle)
            self.handle = None


__all__ = ["Device", "Tables", "FP16Keys", "PackedKeys", "CompressedKeys", "Values", "append_count",
           "RangeError", "StateError"]
