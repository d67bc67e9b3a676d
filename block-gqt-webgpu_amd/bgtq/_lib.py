"""ctypes binding of libbgtq.so (include/bgtq.h).

The library is required: there is no CPU fallback. Import succeeds without a
GPU (the symbols load); calls that need a device fail with DeviceError.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("BGTQ_LIB", Path(__file__).resolve().parent.parent / "lib" / "libbgtq.so"))

OK, ERR_RANGE, ERR_STATE, ERR_DEVICE, ERR_UNSUPPORTED, ERR_NOMEM = range(6)
DTYPE_F32, DTYPE_F16 = 0, 1
KEYS_FP16, KEYS_PACKED, KEYS_COMPRESSED = 0, 1, 2
ROLES = {0: "persistent-k", 1: "persistent-v", 2: "shared", 3: "scratch"}


class RangeError(ValueError):
    """The reference's RangeError: an invalid argument, no state changed."""


class StateError(RuntimeError):
    """The reference's Error: an invalid object state, no state changed."""


class DeviceError(RuntimeError):
    """HIP runtime failure."""


class UnsupportedError(NotImplementedError):
    """Valid input this build does not handle."""


class TablesInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "groups", "row_bytes", "norm_stride", "nibble_dims",
                                             "max_centroids", "n_codebooks", "n_books")] + [
        ("device_bytes", ctypes.c_uint64)]


class Allocation(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("role", ctypes.c_int32), ("bytes", ctypes.c_uint64)]


class EncodeJob(ctypes.Structure):
    _fields_ = [("tables", ctypes.c_void_p), ("src", ctypes.c_void_p), ("src_row_stride", ctypes.c_int64),
                ("rows", ctypes.c_int64), ("packed", ctypes.c_void_p), ("norms", ctypes.c_void_p),
                ("dst_row0", ctypes.c_int64)]


class DecodeDesc(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("q_heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
                ("dim", ctypes.c_int32), ("key_format", ctypes.c_int32), ("tables", ctypes.c_void_p * 16),
                ("packed", ctypes.c_void_p), ("packed_seq_stride", ctypes.c_int64),
                ("packed_head_stride", ctypes.c_int64), ("norms", ctypes.c_void_p),
                ("norms_seq_stride", ctypes.c_int64), ("norms_head_stride", ctypes.c_int64),
                ("k_f16", ctypes.c_void_p), ("k_seq_stride", ctypes.c_int64), ("k_head_stride", ctypes.c_int64),
                ("v", ctypes.c_void_p), ("v_dtype", ctypes.c_int32), ("v_seq_stride", ctypes.c_int64),
                ("v_head_stride", ctypes.c_int64), ("q", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("lengths", ctypes.c_void_p), ("max_length", ctypes.c_uint32), ("splits", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("q_rotated", ctypes.c_int32)]



class AppendDesc(ctypes.Structure):
    _fields_ = [("k_new", ctypes.c_void_p), ("k_new_dtype", ctypes.c_int32), ("k_new_seq_stride", ctypes.c_int64),
                ("k_new_head_stride", ctypes.c_int64), ("v_new", ctypes.c_void_p), ("v_new_dtype", ctypes.c_int32),
                ("v_new_seq_stride", ctypes.c_int64), ("v_new_head_stride", ctypes.c_int64)]


class PrefillAppendDesc(ctypes.Structure):
    _fields_ = [("k_new", ctypes.c_void_p), ("k_new_dtype", ctypes.c_int32), ("k_new_seq_stride", ctypes.c_int64),
                ("k_new_row_stride", ctypes.c_int64), ("k_new_head_stride", ctypes.c_int64),
                ("v_new", ctypes.c_void_p), ("v_new_dtype", ctypes.c_int32), ("v_new_seq_stride", ctypes.c_int64),
                ("v_new_row_stride", ctypes.c_int64), ("v_new_head_stride", ctypes.c_int64)]


class PrefillDesc(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("rows", ctypes.c_int32), ("q_heads", ctypes.c_int32),
                ("kv_heads", ctypes.c_int32), ("dim", ctypes.c_int32), ("key_format", ctypes.c_int32),
                ("tables", ctypes.c_void_p * 16), ("packed", ctypes.c_void_p), ("packed_seq_stride", ctypes.c_int64),
                ("packed_head_stride", ctypes.c_int64), ("norms", ctypes.c_void_p),
                ("norms_seq_stride", ctypes.c_int64), ("norms_head_stride", ctypes.c_int64),
                ("k_f16", ctypes.c_void_p), ("k_seq_stride", ctypes.c_int64), ("k_head_stride", ctypes.c_int64),
                ("v", ctypes.c_void_p), ("v_seq_stride", ctypes.c_int64), ("v_head_stride", ctypes.c_int64),
                ("q", ctypes.c_void_p), ("out", ctypes.c_void_p), ("starts", ctypes.c_void_p),
                ("max_length", ctypes.c_uint32), ("split_tokens", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("q_rotated", ctypes.c_int32)]

class Binding(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_size_t), ("tables", ctypes.c_void_p)]


class ModelDispatch(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("params", ctypes.c_uint32 * 8), ("bindings", ctypes.POINTER(Binding)),
                ("n_bindings", ctypes.c_size_t), ("x", ctypes.c_uint32), ("y", ctypes.c_uint32)]


class GroupTables(ctypes.Structure):
    _fields_ = [("centroids", ctypes.c_void_p), ("rotation", ctypes.c_void_p)]


_VP, _SZ, _I32, _U32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint32
_PP = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "bgtq_last_error": (ctypes.c_char_p, []),
    "bgtq_abi_version": (_I32, []),
    "bgtq_context_create": (_I32, [_I32, _PP]),
    "bgtq_context_destroy": (None, [_VP]),
    "bgtq_context_synchronize": (_I32, [_VP]),
    "bgtq_context_stream": (_VP, [_VP]),
    "bgtq_context_set_stream": (_I32, [_VP, _VP]),
    "bgtq_timestamps_create": (_I32, [_VP, _U32, _PP]),
    "bgtq_timestamps_write": (_I32, [_VP, _U32]),
    "bgtq_timestamps_resolve": (_I32, [_VP, _U32, _U32, ctypes.POINTER(ctypes.c_uint64)]),
    "bgtq_timestamps_destroy": (None, [_VP]),
    "bgtq_tables_create": (_I32, [_VP, _VP, _SZ, _VP, _SZ, _PP]),
    "bgtq_tables_info_get": (_I32, [_VP, ctypes.POINTER(TablesInfo)]),
    "bgtq_tables_destroy": (None, [_VP]),
    "bgtq_fp16_keys_create": (_I32, [_VP, _U32, _U32, _PP]),
    "bgtq_packed_keys_create": (_I32, [_VP, _U32, _PP]),
    "bgtq_compressed_keys_create": (_I32, [_VP, _U32, _PP]),
    "bgtq_keys_append": (_I32, [_VP, _VP, _SZ]),
    "bgtq_keys_ready": (_I32, [_VP]),
    "bgtq_keys_kind": (_I32, [_VP]),
    "bgtq_keys_length": (_U32, [_VP]),
    "bgtq_keys_capacity": (_U32, [_VP]),
    "bgtq_keys_dim": (_U32, [_VP]),
    "bgtq_keys_read_packed": (_I32, [_VP, _VP, _SZ, _VP, _SZ]),
    "bgtq_keys_read_fp16": (_I32, [_VP, _VP, _SZ]),
    "bgtq_keys_prepare": (_I32, [_VP, _VP, _SZ]),
    "bgtq_keys_allocations": (_I32, [_VP, _VP, _SZ, ctypes.POINTER(ctypes.c_size_t)]),
    "bgtq_keys_destroy": (None, [_VP]),
    "bgtq_values_create": (_I32, [_VP, _U32, _U32, _I32, _PP]),
    "bgtq_values_append": (_I32, [_VP, _VP, _SZ]),
    "bgtq_values_length": (_U32, [_VP]),
    "bgtq_values_allocations": (_I32, [_VP, _VP, _SZ, ctypes.POINTER(ctypes.c_size_t)]),
    "bgtq_values_destroy": (None, [_VP]),
    "bgtq_attention_create": (_I32, [_VP, _VP, _U32, _I32, _PP]),
    "bgtq_attention_set_queries": (_I32, [_VP, _VP, _SZ, _VP, _SZ, _I32]),
    "bgtq_attention_record": (_I32, [_VP]),
    "bgtq_attention_record_timed": (_I32, [_VP, _VP, _U32, _U32]),
    "bgtq_attention_attend": (_I32, [_VP, _VP, _SZ, _VP, _SZ, _I32]),
    "bgtq_attention_read": (_I32, [_VP, _I32, _VP, _SZ]),
    "bgtq_attention_queries": (_U32, [_VP]),
    "bgtq_attention_allocations": (_I32, [_VP, _VP, _SZ, ctypes.POINTER(ctypes.c_size_t)]),
    "bgtq_attention_destroy": (None, [_VP]),
    "bgtq_encode_batched": (_I32, [_VP, _I32, ctypes.POINTER(EncodeJob), _SZ]),
    "bgtq_decode_workspace_size": (_I32, [ctypes.POINTER(DecodeDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "bgtq_decode": (_I32, [_VP, ctypes.POINTER(DecodeDesc)]),
    "bgtq_decode_append": (_I32, [_VP, ctypes.POINTER(DecodeDesc), ctypes.POINTER(AppendDesc)]),
    "bgtq_decode_noalloc": (_I32, [_VP, ctypes.POINTER(DecodeDesc)]),
    "bgtq_bake_qproj": (_I32, [_VP, ctypes.c_size_t, _VP, ctypes.c_size_t, ctypes.c_int32, ctypes.c_int64, _VP, _VP,
                               _VP, _VP]),
    "bgtq_prefill_workspace_size": (_I32, [ctypes.POINTER(PrefillDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "bgtq_prefill": (_I32, [_VP, ctypes.POINTER(PrefillDesc)]),
    "bgtq_prefill_append": (_I32, [_VP, ctypes.POINTER(PrefillDesc), ctypes.POINTER(PrefillAppendDesc)]),
    "bgtq_model_submit": (_I32, [_VP, ctypes.POINTER(ModelDispatch), _SZ]),
    "bgtq_allocate_bits": (_I32, [_VP, _SZ, ctypes.c_int64, _I32, _I32, _VP]),
    "bgtq_layout_groups": (_I32, [_VP, _SZ, _VP, _VP, _VP]),
    "bgtq_layout_build": (_I32, [_VP, _SZ, ctypes.POINTER(GroupTables), _SZ, _I32, _I32, _VP,
                                 ctypes.POINTER(ctypes.c_size_t), _VP, ctypes.POINTER(ctypes.c_size_t)]),
}

_lib = None


def lib():
    """Load libbgtq.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with python block-gqt-webgpu_amd/build.py")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int):
    if status == OK:
        return
    msg = lib().bgtq_last_error().decode()
    raise {ERR_RANGE: RangeError, ERR_STATE: StateError, ERR_UNSUPPORTED: UnsupportedError}.get(
        status, DeviceError)(msg)


def ptr(a):
    """Address of a numpy array's data (None for None)."""
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def allocations(fn, handle):
    n = ctypes.c_size_t(0)
    check(fn(handle, None, 0, ctypes.byref(n)))
    arr = (Allocation * max(1, n.value))()
    check(fn(handle, ctypes.cast(arr, ctypes.c_void_p), n.value, ctypes.byref(n)))
    return [{"name": a.name.decode(), "role": ROLES[a.role], "bytes": int(a.bytes)} for a in arr[:n.value]]
