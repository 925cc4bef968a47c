import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "xmetai-onnx-plugins_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # Flush a line naming each GPU test before it runs, so a run that loses the
    # device still says which case was executing.
    for item in items:
        if item.get_closest_marker("gpu") is not None:
            item.add_marker(pytest.mark.usefixtures("_announce_gpu_case"))


@pytest.fixture(params=["chunk", "seq"])
def m3_path(request, monkeypatch):
    """Mamba3SisoFn kernel under test: the chunked fp32-MFMA kernel (default)
    or the token-by-token kernel (XM_M3_PATH=seq)."""
    if request.param == "seq":
        monkeypatch.setenv("XM_M3_PATH", "seq")
    else:
        monkeypatch.delenv("XM_M3_PATH", raising=False)
    return request.param


@pytest.fixture
def _announce_gpu_case(request):
    sys.stdout.write(f"\n[gpu case] {request.node.nodeid}\n")
    sys.stdout.flush()
    yield
