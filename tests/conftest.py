import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gfx950_available() -> bool:
    try:
        import torch
    except Exception:  # noqa: BLE001
        return False
    if not torch.cuda.is_available():
        return False
    name = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
    return name.startswith("gfx950")


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a gfx950 device is present; fail loudly if the library is not built."""
    if not gfx950_available():
        pytest.skip("needs a gfx950 (MI355X) device")
    from sglang_restomod_amd.attention.mi355x import _lib

    _lib.load()  # raises if the .so is missing: no silent fallback
    import torch

    return torch.device("cuda:0")
