import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libdsa_hip.so")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from cppmega_amd import _lib
    from cppmega_amd.build_lib import deps
    lib_mtime = os.path.getmtime(_lib.LIB_PATH)
    stale = [s for s in deps() if os.path.getmtime(s) > lib_mtime + 1]
    assert not stale, f"libdsa_hip.so is older than {stale}: rebuild before running GPU tests"
    _lib.load()
    return torch.device("cuda", 0)
