"""Copy the reference's committed golden data files into tests/golden/reference.

The files are data (JSON manifests plus little-endian payloads, each checked by
its own sha256); nothing from the reference's source is copied. Run once in a
container where the reference checkout exists:

    python tests/golden/import_reference_fixtures.py /root/reference
"""
import hashlib
import json
import shutil
import sys
from pathlib import Path

WANTED = ["allocator.json", "mixed", "attention", "model/calibration.json", "model/calibration.bin", "model/rope.json",
          "model/rope.bin"]


def main(src):
    src = Path(src) / "fixtures"
    dst = Path(__file__).resolve().parent / "reference"
    for item in WANTED:
        s = src / item
        files = sorted(s.iterdir()) if s.is_dir() else [s]
        for f in files:
            target = dst / f.relative_to(src)
            target.parent.mkdir(parents=True, exist_ok=True)
            shutil.copyfile(f, target)
    for manifest in dst.rglob("*.json"):
        meta = json.loads(manifest.read_text())
        if "binary" in meta:
            payload = manifest.with_name(meta["binary"]).read_bytes()
            assert hashlib.sha256(payload).hexdigest() == meta["sha256"], manifest
    print("copied", sum(1 for _ in dst.rglob("*") if _.is_file()), "files")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
