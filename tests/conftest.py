import json
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

os.environ.setdefault("MICA_AMD_STRICT", "1")  # a kernel miss in a test is an error, never a fallback


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmica_amd.so")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def kat():
    return json.loads((ROOT / "tests" / "golden" / "kat_w8a8.json").read_text())


@pytest.fixture(scope="session")
def gpu():
    """The GPU device, with the kernels verified to be loadable; skips nothing -- a gpu-marked test
    on a machine without the GPU or the library fails loudly."""
    import torch

    from mica_amd import int8_kernels

    ok, why = int8_kernels.available("cuda")
    assert ok, f"mica_amd kernels unavailable: {why}"
    return torch.device("cuda", torch.cuda.current_device())
