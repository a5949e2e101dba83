import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# Copy-engine mode hands transfers under 32 MiB to the zero-copy kernel; the
# parity tests use small shapes and must reach the SDMA path itself.
os.environ["FLEXKV_CE_MIN_BYTES"] = "0"
# Layer-wise host caches with scattered ids move with the zero-copy kernel by
# default; the parity suite keeps their copy-engine form (one SDMA rect copy
# per block) in play.  test_rect_policy_default checks the default itself.
os.environ["FLEXKV_CE_RECT_COPIES"] = "1"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(autouse=True)
def _skip_gpu_without_device(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("no HIP device")


@pytest.fixture(params=["compiled", "ctypes"])
def per_call_path(request, monkeypatch):
    """Run a test through the compiled per-call module of c_ext and through
    the ctypes calls that stand in for it when the module cannot be imported."""
    from flexkv_amd import _lib
    monkeypatch.setenv("FLEXKV_PY_FASTCALL", "0" if request.param == "ctypes" else "1")
    _lib.reset_fast()
    fast = _lib.fast()
    assert isinstance(fast, _lib._CtypesCalls) == (request.param == "ctypes")
    yield request.param
    monkeypatch.delenv("FLEXKV_PY_FASTCALL")
    _lib.reset_fast()
