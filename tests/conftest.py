import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle_ffi import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle_ffi import Reference, reference_available
    if not reference_available():
        pytest.skip("oracle/_ref (picchio built from /root/reference) not present")
    return Reference()


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no GPU")
    import picchio_amd
    picchio_amd.lib()          # the native path must load; no fallback
    return True
