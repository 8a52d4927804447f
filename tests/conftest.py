import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def kvops():
    """The launch module, initialised on device 0 (GPU tests only)."""
    if not gpu_available():
        pytest.fail("GPU test run without a GPU")
    import kv_offload_proto_amd
    from kv_offload_proto_amd.kvops_ext import _kvops

    try:
        _kvops.init(0, "")
    except RuntimeError as exc:
        if "already inited" not in str(exc):
            raise
    return _kvops
