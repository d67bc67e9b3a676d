"""Build libbgtq.so (HIP kernels for gfx950 + the C ABI) in place.

    python block-gqt-webgpu_amd/build.py            # library
    python block-gqt-webgpu_amd/build.py --napi     # library + Node N-API addon

hipcc cross-compiles for gfx950 without a GPU present. All device code is
built with -ffp-contract=off (the encoder reproduces a CPU rounding sequence
bit for bit, so nothing may be fused behind its back), correctly rounded fp32
division/square root, FP32 denormals kept, and packed-FP32 instruction
selection disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
OBJ_DIR = PKG / "_build"
INCLUDE = PKG.parent / "include"
ARCH = os.environ.get("BGTQ_OFFLOAD_ARCH", "gfx950")

DEVICE_SOURCES = ["encode.hip", "encode_bulk.hip", "encode_wave.hip", "decode.hip", "decode_fast.hip",
                  "decode_fast_any64.hip", "decode_fast_any64_append.hip", "decode_fast_any64_prefill.hip",
                  "decode_fast_any128.hip",
                  "decode_fast_d64.hip", "decode_fast_d64_append.hip", "decode_fast_d64_prefill.hip",
                  "decode_fast_d128.hip", "prefill.hip", "reconstruct.hip", "model_ops.hip", "decode_scratch.hip"]
HOST_SOURCES = ["bgtq_api.cpp", "calibrate.cpp"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}"]
# -amdgpu-mfma-vgpr-form: matrix-core accumulators in ordinary VGPRs (gfx950's
# unified register file), so the softmax rescale of the output accumulators
# needs no copies between accumulation and architectural registers.
DEVICE_FLAGS = [f"--offload-arch={ARCH}", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
                "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form"]

# Per-source additions. prefill.hip: its attention inputs are finite, so the
# maxima of matrix-core results need no IEEE NaN quieting (one extra VALU
# instruction per operand otherwise). The fused decode kernel's kinds of launch
# take the machine scheduler that measured best for each (A/B on one box,
# the other units keep the default):
#   decode_fast_d64.hip (decode, structured layouts): max-ilp, C5 layout B
#     6350 -> 6380 GB/s;
#   decode_fast_any64.hip (decode, any packed layout): max-ilp, C5 on the
#     SmolLM2 calibration heads 5379 -> 5445 GB/s;
#   decode_fast_d64_append.hip (decode with an appended token): max-ilp and
#     wave priorities raised around the memory-issue phase, the SmolLM2 step
#     (layout B) 248.6 -> 243.4 us;
#   decode_fast_any64_append.hip (the same on any packed layout): max-memory-
#     clause, the SmolLM2 step on its calibration heads 301.6 -> 296.2 us.
# (Row-wise prefill measured up to 1% slower under these and the tiled
# prefill no different: both keep the default.)
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {"prefill.hip": ["-fno-honor-nans"],
                "decode_fast_d64.hip": _MAX_ILP,
                "decode_fast_any64.hip": _MAX_ILP,
                "decode_fast_d64_append.hip": _MAX_ILP + ["-mllvm", "-amdgpu-set-wave-priority"],
                "decode_fast_any64_append.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the packed-fp32 target feature; drop that noise.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    return err


def build_library(verbose=False) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    jobs = []
    for src in DEVICE_SOURCES:
        jobs.append([cc, *COMMON, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o",
                     str(OBJ_DIR / (src + ".o"))])
    for src in HOST_SOURCES:
        jobs.append([cc, *COMMON, f"--offload-arch={ARCH}", "-c", str(CSRC / src), "-o", str(OBJ_DIR / (src + ".o"))])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out:
                print(out, file=sys.stderr)
    target = LIB_DIR / "libbgtq.so"
    tmp = LIB_DIR / "libbgtq.so.tmp"
    objs = [str(OBJ_DIR / (s + ".o")) for s in DEVICE_SOURCES + HOST_SOURCES]
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs])
    os.replace(tmp, target)
    return target


def build_probes() -> Path:
    """libbgtq_probes.so: the benchmark's streaming-read and matrix-core ceiling kernels."""
    LIB_DIR.mkdir(exist_ok=True)
    target = LIB_DIR / "libbgtq_probes.so"
    tmp = LIB_DIR / "libbgtq_probes.so.tmp"
    _run([hipcc(), *COMMON, *DEVICE_FLAGS, "-shared", "-o", str(tmp), str(CSRC / "probes.hip")])
    os.replace(tmp, target)
    return target


def build_napi() -> Path:
    """Node N-API addon over libbgtq.so (headers from the image's Node)."""
    node_inc = None
    for cand in ("/usr/include/node", "/usr/local/include/node"):
        if (Path(cand) / "node_api.h").exists():
            node_inc = cand
    if node_inc is None:
        raise RuntimeError("node_api.h not found")
    src = PKG / "node" / "bgtq_napi.cc"
    out = PKG / "node" / "bgtq_napi.node"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-DNAPI_VERSION=6", f"-I{node_inc}", f"-I{INCLUDE}",
          str(src), "-o", str(out), f"-L{LIB_DIR}", "-lbgtq", "-Wl,-rpath,$ORIGIN/../lib"])
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--napi", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build_library(a.verbose))
    print(build_probes())
    if a.napi:
        print(build_napi())


if __name__ == "__main__":
    main()
