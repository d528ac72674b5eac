import json
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def fixtures():
    with open(GOLDEN / "reference_fixtures.json") as f:
        return json.load(f)


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (not skip) without one, so a silent pass is impossible."""
    import torch

    assert torch.cuda.is_available(), "GPU test requires an available MI355X"
    from llm_infer_rust_amd import _native

    _native.lib()  # the HIP library must load; no fallback exists
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before each GPU step so a hang or fault can be attributed.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield


os.environ.setdefault("PYTHONHASHSEED", "0")
