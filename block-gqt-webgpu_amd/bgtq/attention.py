"""Attention sessions: AttentionEngine/AttentionSession and OptimizedAttention.

Mirrors src/attention/attention.ts:6-70 (phase 3: FP16 or materialised FP32
K) and src/attention/optimized.ts:5-45 (phase 4: packed K rebuilt on chip).
setQueries validates with the reference's messages; attend() runs and waits;
inspect() returns logits, probabilities and output read back from the device
(materialised unless the session was created with materialize=False).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib, ptr


class _Session:
    def __init__(self, keys, values, max_queries: int, materialize: bool = True):
        if not isinstance(max_queries, (int, np.integer)):
            raise _lib.RangeError("Incompatible attention storage")
        h = ctypes.c_void_p()
        check(lib().bgtq_attention_create(keys.handle, values.handle, int(max_queries), int(bool(materialize)),
                                          ctypes.byref(h)))
        self.handle, self.keys, self.values, self.maxQueries = h, keys, values, int(max_queries)
        self.materialize = bool(materialize)

    @property
    def allocations(self):
        return _lib.allocations(lib().bgtq_attention_allocations, self.handle)

    def setQueries(self, q, positions, causal: bool = False) -> None:
        qa = np.ascontiguousarray(np.asarray(q, dtype=np.float32).reshape(-1))
        pa = np.ascontiguousarray(np.asarray(positions, dtype=np.uint32).reshape(-1))
        check(lib().bgtq_attention_set_queries(self.handle, ptr(qa), qa.size, ptr(pa), pa.size, int(bool(causal))))

    def record(self, timestamps=None, begin_index: int = 0, end_index: int = 1) -> None:
        """record(encoder, timestamps?) (src/attention/attention.ts:44-58): with
        a Timestamps set, begin_index is written right before the attention
        work and end_index right after it."""
        if timestamps is None:
            check(lib().bgtq_attention_record(self.handle))
        else:
            check(lib().bgtq_attention_record_timed(self.handle, timestamps.handle, int(begin_index),
                                                    int(end_index)))

    def attend(self, q, positions, causal: bool = False) -> np.ndarray:
        """Run attention and return the output [queries, dim] (the GPUBuffer's contents)."""
        qa = np.ascontiguousarray(np.asarray(q, dtype=np.float32).reshape(-1))
        pa = np.ascontiguousarray(np.asarray(positions, dtype=np.uint32).reshape(-1))
        check(lib().bgtq_attention_attend(self.handle, ptr(qa), qa.size, ptr(pa), pa.size, int(bool(causal))))
        return self.read("output")

    def read(self, which: str) -> np.ndarray:
        n = lib().bgtq_attention_queries(self.handle)
        tokens = self.keys.length
        sel = {"logits": 0, "probabilities": 1, "output": 2}[which]
        shape = (n, self.keys.dim) if sel == 2 else (n, tokens)
        out = np.zeros(shape, np.float32)
        check(lib().bgtq_attention_read(self.handle, sel, ptr(out), out.size))
        return out

    def inspect(self) -> dict:
        n = lib().bgtq_attention_queries(self.handle)
        res = {"output": self.read("output"), "queries": n, "tokens": self.keys.length}
        if self.materialize:
            res["logits"] = self.read("logits")
            res["probabilities"] = self.read("probabilities")
        return res

    def destroy(self) -> None:
        if self.handle:
            lib().bgtq_attention_destroy(self.handle)
            self.handle = None


class AttentionSession(_Session):
    """src/attention/attention.ts:19-70 over FP16Keys or CompressedKeys."""


class AttentionEngine:
    """src/attention/attention.ts:6-17."""

    def __init__(self, device):
        self.device = device

    @classmethod
    def create(cls, device):
        return cls(device)

    def session(self, keys, values, maxQueries: int = 3, materialize: bool = True) -> AttentionSession:
        return AttentionSession(keys, values, maxQueries, materialize)


class OptimizedAttention(_Session):
    """src/attention/optimized.ts:5-45 over PackedKeys (fused on-chip K rebuild)."""

    @classmethod
    def create(cls, device, keys, values, maxQueries: int = 3, tailMode: str = "parallel", materialize: bool = True):
        if tailMode not in ("serial", "parallel"):
            raise _lib.RangeError("Unsupported tail mode")
        s = cls(keys, values, maxQueries, materialize)
        s.tailMode = tailMode
        return s
