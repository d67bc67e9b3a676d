"""Calibration tables: BlockGTQParameters, validate_layout, tables.

Mirrors src/webgpu/layout.ts:2-31 (same fields, same checks, same messages,
same serialized integer/float tables). The serialized form is what the C ABI
takes (bgtq_tables_create) and what the model calibration blob stores per
head (src/model/calibration.ts:15-20, tests/oracles/calibrate_model.py:36-41).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import RangeError


@dataclass
class BlockGTQParameters:
    dim: int
    groups: int
    rowBytes: int
    normStride: int
    nibbleDims: int
    maxCentroids: int
    permutation: np.ndarray        # uint32 [dim]
    groupOf: np.ndarray            # uint32 [dim]
    positionToCodebook: np.ndarray  # uint32 [dim]
    codeLut: np.ndarray            # uint8 [n_codebooks*256]
    rotation: np.ndarray           # float32 [dim*dim], y_j = sum_i x_i R[j*dim+i]
    centroids: np.ndarray          # float32 [dim*maxCentroids]
    offsets: np.ndarray            # float32 [dim]
    inverseScales: np.ndarray      # float32 [dim]

    @classmethod
    def from_mixed_fixture(cls, meta, a):
        """The mapping of tests/webgpu/attention-fixture.ts:10-13."""
        if np.any(a["pack_perm"] != np.arange(meta["dim"])):
            raise RangeError("Unsupported secondary permutation")
        return cls(dim=meta["dim"], groups=meta["n_groups"], rowBytes=meta["row_bytes"],
                   normStride=meta["norm_stride"], nibbleDims=meta["nopack_start"],
                   maxCentroids=meta["max_centroids"], permutation=a["head_perm"], groupOf=a["group_of"],
                   positionToCodebook=a["pos_to_cb"], codeLut=a["code_lut"], rotation=a["rotation"],
                   centroids=a["centroids"], offsets=a["lut_offsets"], inverseScales=a["lut_inv_scales"])

    @classmethod
    def load_mixed_fixture(cls, path):
        """A calibration fixture file (JSON manifest plus its little-endian
        payload, tests/webgpu/fixture.ts) read into parameters: loadFixture
        and the mapping of tests/webgpu/attention-fixture.ts:6-13."""
        import hashlib
        import json
        from pathlib import Path
        path = Path(path)
        meta = json.loads(path.read_text(encoding="utf-8"))
        if meta.get("endianness") != "little":
            raise RangeError("Unsupported fixture format")
        payload = path.with_name(meta["binary"]).read_bytes()
        if len(payload) != meta["byte_length"] or hashlib.sha256(payload).hexdigest() != meta["sha256"]:
            raise RangeError("Fixture payload length/hash mismatch")
        kinds = {"f32": "<f4", "u32": "<u4", "u8": "u1", "f16": "<f2", "u16": "<u2"}
        arrays = {}
        for name, d in meta["arrays"].items():
            dt = np.dtype(kinds[d["dtype"]])
            arrays[name] = np.frombuffer(payload, dt, d["nbytes"] // dt.itemsize, d["offset"]).reshape(d["shape"])
        return cls.from_mixed_fixture(meta, arrays)

    @classmethod
    def from_serialized(cls, integer, floating):
        """Inverse of tables(): read a model calibration blob (config, table)."""
        c = np.asarray(integer, dtype=np.int64)
        d, mc = int(c[0]), int(c[5])
        t = np.asarray(floating, dtype=np.float32)
        off = d * d + d * mc
        return cls(dim=d, groups=int(c[1]), rowBytes=int(c[2]), normStride=int(c[3]), nibbleDims=int(c[4]),
                   maxCentroids=mc, permutation=c[c[6]:c[6] + d], groupOf=c[c[7]:c[7] + d],
                   positionToCodebook=c[c[8]:c[8] + d], codeLut=c[c[9]:].astype(np.uint8),
                   rotation=t[:d * d], centroids=t[d * d:off], offsets=t[off:off + d],
                   inverseScales=t[off + d:off + 2 * d])


def validate_layout(p: BlockGTQParameters) -> None:
    """src/webgpu/layout.ts:8-23."""
    d = p.dim
    ints = [d, p.groups, p.rowBytes, p.normStride, p.nibbleDims, p.maxCentroids]
    if (not all(isinstance(v, (int, np.integer)) for v in ints) or d < 2 or d > 128 or d % 2 or p.groups < 1
            or p.groups > 8 or p.normStride < p.groups or p.nibbleDims < 0 or p.nibbleDims > d
            or p.nibbleDims % 2 or p.rowBytes < p.nibbleDims // 2 + d - p.nibbleDims or p.maxCentroids < 2
            or p.maxCentroids > 256):
        raise RangeError("Invalid Block-GTQ layout")
    perm = np.asarray(p.permutation).reshape(-1)
    grp = np.asarray(p.groupOf).reshape(-1)
    cb = np.asarray(p.positionToCodebook).reshape(-1)
    lut = np.asarray(p.codeLut).reshape(-1)
    if (len(perm) != d or len(set(perm.tolist())) != d or np.any(perm >= d) or len(grp) != d
            or np.any(grp >= p.groups) or len(cb) != d or np.asarray(p.rotation).size != d * d
            or np.asarray(p.centroids).size != d * p.maxCentroids or np.asarray(p.offsets).size != d
            or np.asarray(p.inverseScales).size != d or len(lut) % 256 or np.any(cb * 256 >= len(lut))):
        raise RangeError("Invalid calibration table shape")
    for values in (p.rotation, p.centroids, p.offsets, p.inverseScales):
        if not np.all(np.isfinite(np.asarray(values, dtype=np.float32))):
            raise RangeError("Nonfinite calibration table")
    codes = lut.reshape(-1, 256)[cb]  # [d, 256]
    if np.any(codes >= p.maxCentroids) or np.any(codes[:p.nibbleDims] > 15):
        raise RangeError("Code LUT incompatible with packing")


def tables(p: BlockGTQParameters):
    """src/webgpu/layout.ts:24-31 -> (integer uint32[], floating float32[])."""
    validate_layout(p)
    config = [p.dim, p.groups, p.rowBytes, p.normStride, p.nibbleDims, p.maxCentroids, 0, 0, 0, 0]
    for slot, values in ((6, p.permutation), (7, p.groupOf), (8, p.positionToCodebook), (9, p.codeLut)):
        config[slot] = len(config)
        config.extend(int(v) for v in np.asarray(values).reshape(-1))
    integer = np.asarray(config, dtype=np.uint32)
    floating = np.concatenate([np.asarray(a, dtype=np.float32).reshape(-1)
                               for a in (p.rotation, p.centroids, p.offsets, p.inverseScales)])
    return integer, floating
