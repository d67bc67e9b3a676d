import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "block-gqt-webgpu_amd"))
GOLDEN = ROOT / "tests" / "golden"
REF = GOLDEN / "reference"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not O.LIB_PATH.exists():
        O.build()
    return O


@pytest.fixture(scope="session")
def device():
    import bgtq
    dev = bgtq.Device(0)
    yield dev
    dev.destroy()


@pytest.fixture(scope="session")
def mixed_cases(oracle):
    import json
    index = json.loads((REF / "mixed" / "index.json").read_text())["cases"]
    return [(c["name"],) + oracle.read_fixture(REF / "mixed" / f"{c['name']}.json") for c in index]


@pytest.fixture(scope="session")
def attention_cases(oracle):
    import json
    index = json.loads((REF / "attention" / "index.json").read_text())["cases"]
    out = []
    for c in index:
        m, a = oracle.read_fixture(REF / "attention" / f"{c['name']}.json")
        lm, la = oracle.read_fixture(REF / "mixed" / f"{m['layout']}.json")
        assert lm["sha256"] == m["layout_sha256"]
        out.append((c["name"], m, a, lm, la))
    return out
