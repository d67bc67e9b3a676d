"""The Node drop-in (N-API addon + the reference's runtime classes in JS) on the GPU.

Runs block-gqt-webgpu_amd/node/test_napi.js in a child process: the reference's
optimized-attention flow (tests/webgpu/optimized-test.ts:18-45) on committed
golden workloads, packed bytes bit-exact, outputs within the fixture
tolerance, rejections with the reference's messages.
"""
import shutil
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

NODE_DIR = ROOT / "block-gqt-webgpu_amd" / "node"


def test_node_dropin_classes():
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    assert (NODE_DIR / "bgtq_napi.node").exists(), "N-API addon not built (python block-gqt-webgpu_amd/build.py --napi)"
    print("node drop-in test", flush=True)
    r = subprocess.run([node, str(NODE_DIR / "test_napi.js")], capture_output=True, text=True, timeout=180)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
