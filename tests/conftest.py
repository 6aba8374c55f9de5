import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "evo.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # torch first: libevo_hip.so then binds to torch's HIP runtime (same
    # soname), so one runtime owns every device pointer and stream.
    import torch  # noqa: F401


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    if not os.path.exists(oracle_lib.ORACLE_PATH):
        pytest.fail("oracle/liboracle.so is not built: run __graft_entry__.build()")
    return oracle_lib.lib()


@pytest.fixture(scope="session")
def native():
    from evo_hip import native as n
    return n.load()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _release_device_tensors(request):
    yield
    if request.node.get_closest_marker("gpu") is not None:
        import gpu_util
        gpu_util.release()
