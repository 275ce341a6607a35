import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    return pyoracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's own compiled x86 kernels (oracle/_ref), or skip."""
    import pyoracle
    r = pyoracle.load_ref()
    if r is None:
        pytest.skip("oracle/_ref/libqref.so not built (needs the reference sources)")
    return r


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import qwen35_amd
    lib = qwen35_amd.load()
    rc = lib.qhip_init(0)
    assert rc == 0, f"qhip_init failed: {rc}"
    return torch.device("cuda:0")
