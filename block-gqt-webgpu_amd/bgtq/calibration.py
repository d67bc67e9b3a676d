"""Per-(layer, KV head) model calibration tables: the reference's
Calibration.load (src/model/calibration.ts:7-21) over libbgtq tables.

The on-disk format is the reference's fixture format written by its
calibration exporter (tests/oracles/calibrate_model.py:36-49): a JSON
manifest (`calibration.json`) naming a little-endian payload, with per head i
the arrays `h{i}_config` (u32, the tables(p) integer blob), `h{i}_table` (f32,
the float blob) and `h{i}_ranges` (u32, each position's group range). The
checks and their messages follow the reference; a failure raises StateError,
the reference's Error, and leaves nothing allocated.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from ._lib import StateError

# src/model/calibration.ts:10-11: the pinned upstream commit, and the model
# revision required when no adapter is given (the SmolLM2 calibration).
UPSTREAM_COMMIT = "3fe14e7d4b8a6c85402818f7e22052527ed42e93"
DEFAULT_MODEL_REVISION = "12fd25f77366fa6b3b4b768ec3050bf629380bac"
DEFAULT_HEADS = 90  # 30 layers x 3 KV heads without an adapter


@dataclass
class CalibrationBlob:
    """Host copy of one head's arrays."""
    config: np.ndarray  # u32
    table: np.ndarray   # f32
    ranges: np.ndarray  # u32 [64 * 2]

    @property
    def row_bytes(self) -> int:
        return int(self.config[2])

    @property
    def norm_stride(self) -> int:
        return int(self.config[3])


def read(base, layers: int | None = None, kv_heads: int | None = None,
         model_revision: str | None = None) -> tuple[dict, str, list[CalibrationBlob]]:
    """Read and check calibration.json and its payload (no device work).

    layers x kv_heads is the model geometry (the reference's adapter); without
    it 90 heads and the pinned SmolLM2 revision are required."""
    base = Path(base)
    m = json.loads((base / "calibration.json").read_text(encoding="utf-8"))
    payload = (base / m["binary"]).read_bytes()
    sha = hashlib.sha256(payload).hexdigest()
    expected = layers * kv_heads if layers is not None and kv_heads is not None else DEFAULT_HEADS
    revision = model_revision if model_revision is not None else (None if layers is not None else DEFAULT_MODEL_REVISION)
    if (sha != m.get("sha256") or len(m.get("heads", [])) != expected
            or (revision and m.get("model_revision") != revision) or m.get("upstream_commit") != UPSTREAM_COMMIT):
        raise StateError("Calibration mismatch")
    arrays = m.get("arrays", {})

    def array(i, name, dtype):
        a = arrays.get(f"h{i}_{name}")
        if not a or a["offset"] % 4 or a["offset"] + a["nbytes"] > len(payload) or a["nbytes"] % 4:
            raise StateError("Bad calibration descriptor")
        return np.frombuffer(payload, dtype, a["nbytes"] // np.dtype(dtype).itemsize, a["offset"]).copy()

    blobs = []
    for i in range(expected):
        config, table, ranges = array(i, "config", "<u4"), array(i, "table", "<f4"), array(i, "ranges", "<u4")
        if (config.size < 1 or config[0] != 64 or (config.size > 1 and config[1] > 8) or ranges.size != 128
                or not np.isfinite(table).all()):
            raise StateError("Unsupported calibration")
        # rot[k][j] = table[k*64 + j]; entries past a short table count as
        # nonzero, as the reference's out-of-range reads do.
        rot = np.full(64 * 64, np.nan, np.float32)
        rot[:min(table.size, 64 * 64)] = table[:64 * 64]
        rot = rot.reshape(64, 64)
        k = np.arange(64)[:, None]
        lo, hi = ranges[0::2].astype(np.int64)[None, :], ranges[1::2].astype(np.int64)[None, :]
        if np.any(((k < lo) | (k >= hi)) & (rot != 0)):
            raise StateError("Off-group rotation")
        blobs.append(CalibrationBlob(config, table, ranges))
    return m, sha, blobs


@dataclass
class CalibrationHead:
    tables: object  # bgtq.Tables on the device
    ranges: np.ndarray
    row_bytes: int
    norm_stride: int

    # The head's config and table bindings of the model dispatches
    # (src/model/decoder.ts:52, :55): both are its device tables.
    @property
    def config(self):
        return self.tables

    @property
    def table(self):
        return self.tables


class Calibration:
    """Device-resident tables of every (layer, KV head), index layer * kv_heads + head."""

    def __init__(self, device, sha256: str, heads: list[CalibrationHead], meta: dict):
        self.device, self.sha256, self.heads, self.meta = device, sha256, heads, meta

    @classmethod
    def load(cls, device, base, layers: int | None = None, kv_heads: int | None = None,
             model_revision: str | None = None) -> "Calibration":
        from .runtime import Tables
        meta, sha, blobs = read(base, layers, kv_heads, model_revision)
        heads: list[CalibrationHead] = []
        try:
            for b in blobs:
                t = Tables(device, integer=b.config, floating=b.table)
                heads.append(CalibrationHead(t, b.ranges, b.row_bytes, b.norm_stride))
        except Exception:
            for h in heads:
                h.tables.destroy()
            raise
        return cls(device, sha, heads, meta)

    @property
    def allocations(self) -> list[dict]:
        return [{"name": f"head {i} tables", "role": "tables", "bytes": h.tables.info["device_bytes"]}
                for i, h in enumerate(self.heads)]

    def destroy(self) -> None:
        for h in self.heads:
            h.tables.destroy()
        self.heads = []
