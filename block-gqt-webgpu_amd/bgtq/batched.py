"""Batched model-geometry entry points over caller-owned device memory.

Thin wrappers over bgtq_encode_batched / bgtq_decode (include/bgtq.h) that
take torch tensors resident on the GPU (torch supplies device memory and the
stream; all arithmetic runs in libbgtq.so). Used for layers x sequences x KV
heads workloads: the model dispatch sites encode_k / compressed_dot / softmax /
weighted of src/model/decoder.ts:46-56.
"""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import check, lib


def _addr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def bind_torch_stream(device):
    """Order the context's work on torch's current stream."""
    import torch
    device.set_stream(torch.cuda.current_stream().cuda_stream)


def encode(device, jobs, src_dtype="f16"):
    """jobs: iterable of dicts {tables, src, src_row_stride, rows, packed, norms, dst_row0}."""
    jobs = list(jobs)
    arr = (_lib.EncodeJob * max(1, len(jobs)))()
    for i, j in enumerate(jobs):
        arr[i] = _lib.EncodeJob(j["tables"].handle, _addr(j["src"]), int(j["src_row_stride"]), int(j["rows"]),
                                _addr(j["packed"]), _addr(j["norms"]), int(j.get("dst_row0", 0)))
    code = {"f16": _lib.DTYPE_F16, "f32": _lib.DTYPE_F32}[src_dtype]
    check(lib().bgtq_encode_batched(device.handle, code, arr, len(jobs)))


def decode_desc(*, batch, q_heads, kv_heads, dim, q, out, lengths, max_length, v, v_dtype="f16",
                v_seq_stride, v_head_stride, tables=None, packed=None, packed_seq_stride=0,
                packed_head_stride=0, norms=None, norms_seq_stride=0, norms_head_stride=0, k_f16=None,
                k_seq_stride=0, k_head_stride=0, splits=0, workspace=None, q_rotated=False):
    """bgtq_decode_desc over device tensors. q_rotated: q is already R q[perm] per its KV head's
    tables (from a projection baked with calibrate.bake_qproj)."""
    d = _lib.DecodeDesc()
    d.q_rotated = int(bool(q_rotated))
    d.batch, d.q_heads, d.kv_heads, d.dim = batch, q_heads, kv_heads, dim
    d.key_format = _lib.KEYS_PACKED if packed is not None else _lib.KEYS_FP16
    for i, t in enumerate(tables or []):
        d.tables[i] = t.handle.value if hasattr(t.handle, "value") else t.handle
    d.packed, d.packed_seq_stride, d.packed_head_stride = _addr(packed), packed_seq_stride, packed_head_stride
    d.norms, d.norms_seq_stride, d.norms_head_stride = _addr(norms), norms_seq_stride, norms_head_stride
    d.k_f16, d.k_seq_stride, d.k_head_stride = _addr(k_f16), k_seq_stride, k_head_stride
    d.v, d.v_dtype = _addr(v), {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16}[v_dtype]
    d.v_seq_stride, d.v_head_stride = v_seq_stride, v_head_stride
    d.q, d.out, d.lengths = _addr(q), _addr(out), _addr(lengths)
    d.max_length, d.splits = int(max_length), int(splits)
    if workspace is not None:
        d.workspace, d.workspace_bytes = _addr(workspace), workspace.numel() * workspace.element_size()
    return d


def workspace_bytes(desc) -> int:
    n = ctypes.c_size_t(0)
    check(lib().bgtq_decode_workspace_size(ctypes.byref(desc), ctypes.byref(n)))
    return n.value


def decode(device, desc) -> None:
    check(lib().bgtq_decode(device.handle, ctypes.byref(desc)))


def decode_noalloc(device, desc) -> None:
    """bgtq_decode_noalloc: the decode with the library's own device scratch (the descriptor's
    workspace is ignored); nothing is allocated."""
    check(lib().bgtq_decode_noalloc(device.handle, ctypes.byref(desc)))


def append_desc(*, k_new, v_new):
    """bgtq_append_desc over device tensors [B, Hkv, dim] (FP32 or FP16, any strides in elements)."""
    a = _lib.AppendDesc()
    dt = {"torch.float32": _lib.DTYPE_F32, "torch.float16": _lib.DTYPE_F16}
    a.k_new, a.k_new_dtype = _addr(k_new), dt[str(k_new.dtype)]
    a.k_new_seq_stride, a.k_new_head_stride = k_new.stride(0), k_new.stride(1)
    a.v_new, a.v_new_dtype = _addr(v_new), dt[str(v_new.dtype)]
    a.v_new_seq_stride, a.v_new_head_stride = v_new.stride(0), v_new.stride(1)
    return a


def decode_append(device, desc, append) -> None:
    """The decode step with its new token (bgtq_decode_append): row lengths[b] - 1 of the caches."""
    check(lib().bgtq_decode_append(device.handle, ctypes.byref(desc), ctypes.byref(append)))


def prefill_desc(*, batch, rows, q_heads, kv_heads, dim, q, out, starts, max_length, v, v_seq_stride,
                 v_head_stride, tables=None, packed=None, packed_seq_stride=0, packed_head_stride=0, norms=None,
                 norms_seq_stride=0, norms_head_stride=0, k_f16=None, k_seq_stride=0, k_head_stride=0,
                 split_tokens=0, workspace=None, q_rotated=False):
    """bgtq_prefill_desc over device tensors: q/out [B, rows, Hq, dim] FP32, v FP16, starts uint32 [B];
    q_rotated as for decode_desc."""
    d = _lib.PrefillDesc()
    d.q_rotated = int(bool(q_rotated))
    d.batch, d.rows, d.q_heads, d.kv_heads, d.dim = batch, rows, q_heads, kv_heads, dim
    d.key_format = _lib.KEYS_PACKED if packed is not None else _lib.KEYS_FP16
    for i, t in enumerate(tables or []):
        d.tables[i] = t.handle.value if hasattr(t.handle, "value") else t.handle
    d.packed, d.packed_seq_stride, d.packed_head_stride = _addr(packed), packed_seq_stride, packed_head_stride
    d.norms, d.norms_seq_stride, d.norms_head_stride = _addr(norms), norms_seq_stride, norms_head_stride
    d.k_f16, d.k_seq_stride, d.k_head_stride = _addr(k_f16), k_seq_stride, k_head_stride
    d.v, d.v_seq_stride, d.v_head_stride = _addr(v), v_seq_stride, v_head_stride
    d.q, d.out, d.starts = _addr(q), _addr(out), _addr(starts)
    d.max_length, d.split_tokens = int(max_length), int(split_tokens)
    if workspace is not None:
        d.workspace, d.workspace_bytes = _addr(workspace), workspace.numel() * workspace.element_size()
    return d


def prefill_workspace_bytes(desc) -> int:
    n = ctypes.c_size_t(0)
    check(lib().bgtq_prefill_workspace_size(ctypes.byref(desc), ctypes.byref(n)))
    return n.value


def prefill_append_desc(*, k_new, v_new):
    """bgtq_prefill_append_desc over device tensors [B, rows, Hkv, dim] (FP32 or FP16, any strides in
    elements)."""
    a = _lib.PrefillAppendDesc()
    dt = {"torch.float32": _lib.DTYPE_F32, "torch.float16": _lib.DTYPE_F16}
    a.k_new, a.k_new_dtype = _addr(k_new), dt[str(k_new.dtype)]
    a.k_new_seq_stride, a.k_new_row_stride, a.k_new_head_stride = k_new.stride(0), k_new.stride(1), k_new.stride(2)
    a.v_new, a.v_new_dtype = _addr(v_new), dt[str(v_new.dtype)]
    a.v_new_seq_stride, a.v_new_row_stride, a.v_new_head_stride = v_new.stride(0), v_new.stride(1), v_new.stride(2)
    return a


def prefill_append(device, desc, append) -> None:
    """A prefill chunk with its own rows encoded and appended in the same launch (bgtq_prefill_append)."""
    check(lib().bgtq_prefill_append(device.handle, ctypes.byref(desc), ctypes.byref(append)))


def prefill(device, desc) -> None:
    check(lib().bgtq_prefill(device.handle, ctypes.byref(desc)))
