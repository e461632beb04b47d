import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: large checkpoints (hundreds of MiB)")


@pytest.fixture(scope="session")
def ckpt_dir(tmp_path_factory):
    d = os.environ.get("FLOWEDGE_CKPT_DIR")
    if d:
        os.makedirs(d, exist_ok=True)
        return d
    return str(tmp_path_factory.mktemp("ckpt"))


@pytest.fixture(scope="session", autouse=True)
def torch_gpu_first(request):
    """Initialises torch's GPU runtime before any engine exists in a session that runs GPU tests.

    torch (ROCm wheel) fails its first GPU initialisation with "No HIP GPUs are available" when
    it happens after an engine of this library was created and freed in the same process and
    none is alive; initialised earlier, it keeps working.  GPU tests that hand device tensors to
    the C ABI therefore do not depend on which test touched torch's GPU first.
    """
    if any(item.get_closest_marker("gpu") for item in request.session.items):
        import torch

        if torch.cuda.is_available():
            torch.cuda.init()
    yield
