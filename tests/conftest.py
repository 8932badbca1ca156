import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "pjrt-ocl_amd", "python"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvmrt.so)")


@pytest.fixture(scope="session", autouse=True)
def _close_gpu_runtime_at_exit():
    """The GPU tests share one Runtime; close it (programs, pool, stream) at the
    end of the session instead of leaving it to interpreter shutdown."""
    yield
    mod = sys.modules.get("gpu_util")
    if mod is not None:
        mod.close_runtime()
