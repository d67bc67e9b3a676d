"""Block-GTQ CPU oracle, Python side. TEST INFRASTRUCTURE ONLY.

ctypes bindings for oracle/libbgtq_oracle.so (the C restatement of the
reference's Python path) plus a reader for the reference's fixture format
(tests/oracles/fixture.py:33-49). Only tests/, the smoke check and bench.py's
CPU-baseline leg import this module; the product path never does.

Pinning (what checks each function; all in tests/test_oracle.py):
  encode            bit-exact vs fixtures/mixed (10 layouts x 5 rows: codes,
                    raw, corrected, rotated) and fixtures/attention packed_k +
                    norms (1,792 rows); both written by the reference encoder.
  pack/unpack       fixtures/mixed packed bytes + round trip.
  f32_to_f16        the reference's edge probes (tests/test_mixed.py:76-79) and
                    numpy's IEEE conversion over all finite FP16 neighbourhoods.
  reconstruct       fixtures/mixed reconstructed_f32/_f16, fixtures/attention
                    reconstructed_k (within the fixture tolerance).
  attention         fixtures/attention logits/probabilities/output (baseline
                    tolerances), closed forms (zero q -> mean V, causal row 0 ->
                    V0), a float64 numpy softmax.
  allocate_bits     fixtures/allocator.json and the exhaustive small grid of
                    tests/test_allocator.py:24-31 against a brute-force greedy.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libbgtq_oracle.so"

DTYPES = {"f32": np.dtype("<f4"), "u32": np.dtype("<u4"), "u8": np.dtype("u1"),
          "f16": np.dtype("<f2"), "u16": np.dtype("<u2")}

# The reference fixtures were produced on an AVX2 CPU (i5-1235U, torch 2.12
# CPU build, 1 thread): ATen float sums run 8-lane vectors; the sgemm K loop
# is one FMA chain in ascending k.
AVX2 = (8, 0)
AVX512 = (16, 0)


def read_fixture(path):
    """Read a reference fixture (JSON manifest + LE payload), checking sha256."""
    path = Path(path)
    meta = json.loads(path.read_text(encoding="utf-8"))
    if meta["version"] not in (1, 2) or meta["endianness"] != "little":
        raise ValueError("Unsupported fixture format")
    payload = path.with_name(meta["binary"]).read_bytes()
    if len(payload) != meta["byte_length"] or hashlib.sha256(payload).hexdigest() != meta["sha256"]:
        raise ValueError("Fixture payload length/hash mismatch")
    arrays = {}
    for name, desc in meta["arrays"].items():
        dtype = DTYPES[desc["dtype"]]
        expected = int(np.prod(desc["shape"])) * dtype.itemsize
        if desc["offset"] % 4 or desc["nbytes"] != expected or desc["offset"] + expected > len(payload):
            raise ValueError(f"Invalid array descriptor: {name}")
        arrays[name] = np.frombuffer(payload, dtype, expected // dtype.itemsize,
                                     desc["offset"]).reshape(desc["shape"]).copy()
    return meta, arrays


def build():
    """Compile the C oracle in place (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class _Layout(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int32), ("groups", ctypes.c_int32), ("row_bytes", ctypes.c_int32),
                ("norm_stride", ctypes.c_int32), ("nibble_dims", ctypes.c_int32),
                ("max_centroids", ctypes.c_int32), ("n_codebooks", ctypes.c_int32),
                ("perm", ctypes.c_void_p), ("group_of", ctypes.c_void_p), ("pos_to_cb", ctypes.c_void_p),
                ("code_lut", ctypes.c_void_p), ("rotation", ctypes.c_void_p), ("centroids", ctypes.c_void_p),
                ("offsets", ctypes.c_void_p), ("inv_scales", ctypes.c_void_p)]


class _Profile(ctypes.Structure):
    _fields_ = [("sum_lanes", ctypes.c_int32), ("gemm_mode", ctypes.c_int32)]


_lib = None


def use_native_build(out_dir):
    """Build the oracle source for this host's CPU (-O3 -march=native, still no fast-math and no
    contraction: the same results) into out_dir and route every call here through it. The
    benchmark's CPU-baseline leg times it; tests use the portable build."""
    global _lib
    out = Path(out_dir) / "libbgtq_oracle_native.so"
    subprocess.run(["make", "-s", "-C", str(HERE), "native", f"OUT={out}"], check=True)
    _lib = None
    return lib(out)


def lib(path=None):
    global _lib
    if _lib is None:
        if path is None and not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(path or LIB_PATH))
        _lib.bgtq_oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib.bgtq_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.bgtq_oracle_aten_sum.restype = ctypes.c_float
        _lib.bgtq_oracle_aten_sum.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]
        for name in ("bgtq_oracle_encode", "bgtq_oracle_encode_pack", "bgtq_oracle_attention",
                     "bgtq_oracle_attention_f32"):
            getattr(_lib, name).restype = ctypes.c_int32
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


class Layout:
    """Calibration tables (src/webgpu/layout.ts:2-6) held as contiguous numpy arrays."""

    def __init__(self, *, dim, groups, row_bytes, norm_stride, nibble_dims, max_centroids,
                 perm, group_of, pos_to_cb, code_lut, rotation, centroids, offsets, inv_scales):
        self.dim, self.groups, self.row_bytes = int(dim), int(groups), int(row_bytes)
        self.norm_stride, self.nibble_dims, self.max_centroids = int(norm_stride), int(nibble_dims), int(max_centroids)
        u32 = lambda a: np.ascontiguousarray(np.asarray(a).reshape(-1), dtype=np.uint32)
        f32 = lambda a: np.ascontiguousarray(np.asarray(a).reshape(-1), dtype=np.float32)
        self.perm, self.group_of, self.pos_to_cb = u32(perm), u32(group_of), u32(pos_to_cb)
        self.code_lut = np.ascontiguousarray(np.asarray(code_lut).reshape(-1), dtype=np.uint8)
        self.rotation, self.centroids = f32(rotation), f32(centroids)
        self.offsets, self.inv_scales = f32(offsets), f32(inv_scales)
        self._c = _Layout(self.dim, self.groups, self.row_bytes, self.norm_stride, self.nibble_dims,
                          self.max_centroids, len(self.code_lut) // 256, _p(self.perm), _p(self.group_of),
                          _p(self.pos_to_cb), _p(self.code_lut), _p(self.rotation), _p(self.centroids),
                          _p(self.offsets), _p(self.inv_scales))

    @classmethod
    def from_mixed_fixture(cls, meta, a):
        """Same mapping as the reference's tests/webgpu/attention-fixture.ts:10-13."""
        return cls(dim=meta["dim"], groups=meta["n_groups"], row_bytes=meta["row_bytes"],
                   norm_stride=meta["norm_stride"], nibble_dims=meta["nopack_start"],
                   max_centroids=meta["max_centroids"], perm=a["head_perm"], group_of=a["group_of"],
                   pos_to_cb=a["pos_to_cb"], code_lut=a["code_lut"], rotation=a["rotation"],
                   centroids=a["centroids"], offsets=a["lut_offsets"], inv_scales=a["lut_inv_scales"])

    @classmethod
    def from_model_config(cls, config, table):
        """Per-head calibration blob (tests/oracles/model_codec.py:10-15)."""
        c = np.asarray(config, dtype=np.int64)
        d, maxc = int(c[0]), int(c[5])
        t = np.asarray(table, dtype=np.float32)
        off = d * d + d * maxc
        lut = c[int(c[9]):]
        return cls(dim=d, groups=int(c[1]), row_bytes=int(c[2]), norm_stride=int(c[3]), nibble_dims=int(c[4]),
                   max_centroids=maxc, perm=c[int(c[6]):int(c[6]) + d], group_of=c[int(c[7]):int(c[7]) + d],
                   pos_to_cb=c[int(c[8]):int(c[8]) + d], code_lut=lut, rotation=t[:d * d],
                   centroids=t[d * d:off], offsets=t[off:off + d], inv_scales=t[off + d:off + 2 * d])


def f32_to_f16_bits(x):
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    f = lib().bgtq_oracle_f32_to_f16
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def aten_sum(x, lanes=8):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().bgtq_oracle_aten_sum(_p(x), len(x), lanes)


def gemm_abt(a, b, mode=0):
    """a @ b.T with the CPU sgemm K-loop order (mode 0: ascending FMA chain)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros((a.shape[0], b.shape[0]), np.float32)
    lib().bgtq_oracle_gemm_abt(_p(a), _p(b), ctypes.c_int64(a.shape[0]), a.shape[1], b.shape[0], mode, _p(out))
    return out


def encode(layout: Layout, x, profile=AVX2):
    """encode(x, tables) -> codes, raw, corrected, y (production_math.py:4-24)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.shape[0]
    d, ng = layout.dim, layout.groups
    codes = np.zeros((rows, d), np.uint8)
    raw = np.zeros((rows, ng), np.float32)
    corr = np.zeros((rows, ng), np.float32)
    y = np.zeros((rows, d), np.float32)
    prof = _Profile(*profile)
    rc = lib().bgtq_oracle_encode(ctypes.byref(layout._c), ctypes.byref(prof), _p(x), ctypes.c_int64(rows),
                                  _p(codes), _p(raw), _p(corr), _p(y))
    if rc:
        raise ValueError(f"oracle encode failed: {rc}")
    return codes, raw, corr, y


def encode_pack(layout: Layout, k_half_bits, profile=AVX2):
    """Persistent-cache rows for FP16 K: (packed [rows,row_bytes], norm bits [rows,norm_stride])."""
    k = np.ascontiguousarray(k_half_bits, dtype=np.uint16).reshape(-1, layout.dim)
    rows = k.shape[0]
    packed = np.zeros((rows, layout.row_bytes), np.uint8)
    norms = np.zeros((rows, layout.norm_stride), np.uint16)
    prof = _Profile(*profile)
    rc = lib().bgtq_oracle_encode_pack(ctypes.byref(layout._c), ctypes.byref(prof), _p(k), ctypes.c_int64(rows),
                                       _p(packed), _p(norms))
    if rc:
        raise ValueError(f"oracle encode_pack failed: {rc}")
    return packed, norms


def pack(codes, nibble_dims, row_bytes):
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    rows, d = c.reshape(-1, c.shape[-1]).shape
    out = np.zeros((rows, row_bytes), np.uint8)
    lib().bgtq_oracle_pack(_p(c), ctypes.c_int64(rows), d, nibble_dims, row_bytes, _p(out))
    return out.reshape(*c.shape[:-1], row_bytes)


def unpack(packed, dim, nibble_dims):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    rows, rb = p.reshape(-1, p.shape[-1]).shape
    out = np.zeros((rows, dim), np.uint8)
    lib().bgtq_oracle_unpack(_p(p), ctypes.c_int64(rows), dim, nibble_dims, rb, _p(out))
    return out.reshape(*p.shape[:-1], dim)


def reconstruct(layout: Layout, codes, scales):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    rows = codes.shape[0]
    out = np.zeros((rows, layout.dim), np.float32)
    lib().bgtq_oracle_reconstruct(ctypes.byref(layout._c), _p(codes), _p(s), s.shape[1],
                                  ctypes.c_int64(rows), _p(out))
    return out


def attention(q, k, v, positions, causal=False, fp32=False):
    """logits, probabilities, output (src/reference/attention.py:5-22), float64 accumulation;
    fp32=True: the FP32 restatement (the CPU baseline's arithmetic)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    if q.ndim != 2 or k.ndim != 2 or v.ndim != 2 or k.shape != v.shape or q.shape[1] != k.shape[1]:
        raise ValueError("Mismatched or empty attention shapes")
    nq, d = q.shape
    T = k.shape[0]
    if pos.shape != (nq,):
        raise ValueError("One integer position per query is required")
    logits = np.zeros((nq, T), np.float32)
    probs = np.zeros((nq, T), np.float32)
    out = np.zeros((nq, d), np.float32)
    fn = lib().bgtq_oracle_attention_f32 if fp32 else lib().bgtq_oracle_attention
    rc = fn(_p(q), nq, _p(k), _p(v), ctypes.c_int64(T), d, _p(pos), int(bool(causal)), _p(logits), _p(probs), _p(out))
    if rc:
        raise ValueError(f"invalid attention inputs ({rc})")
    return logits, probs, out


def allocate_bits(scores, budget, min_bits=1, max_bits=8):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    w = np.zeros(len(s), np.int64)
    lib().bgtq_oracle_allocate_bits(_p(s) if len(s) else None, len(s), ctypes.c_int64(budget), min_bits, max_bits,
                                    _p(w) if len(s) else None)
    return w


def golden_dir():
    return Path(os.environ.get("BGTQ_GOLDEN", HERE.parent / "tests" / "golden"))
