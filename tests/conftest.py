import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "pure_cuda-c-_frnn_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    if not os.path.exists(os.path.join(ORACLE, "liboracle_frnn.so")):
        subprocess.run(["make", "-C", ORACLE], check=True, stdout=subprocess.DEVNULL)
    yield


def gpu_visible():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


# Count devices once at collection, before any test touches the GPU: a session
# whose first torch.cuda call was is_available() inside a test saw no device
# on the MI355X boxes, while every session that counted devices first did.
gpu_visible()
