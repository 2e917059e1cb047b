import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "pytorch-opt_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import pytest  # noqa: E402
import torch  # noqa: E402

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


# Same device parametrization as the reference suite (tests/conftest.py:4-9);
# the GPU leg carries the gpu mark so `-m gpu` / `-m "not gpu"` split cleanly.
DEVICES = ["cpu"] + ([pytest.param("cuda", marks=pytest.mark.gpu)] if HAS_GPU else [])


@pytest.fixture(params=DEVICES)
def device(request):
    return torch.device(request.param)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP backend. With a GPU present a missing library is a failure,
    never a silent fallback."""
    from pytorch_opt import ops

    assert HAS_GPU, "GPU tests need a visible GPU"
    assert ops.load_native(), "libpytorch_opt_hip.so failed to load"
    return ops._NATIVE


@pytest.fixture
def native_backend(hip):
    from pytorch_opt import ops

    ops.set_backend("native")
    yield hip
    ops.set_backend("auto")
