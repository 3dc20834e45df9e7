import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "nano-hisparse_amd")
for path in (ROOT, PKG_ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libnhs_hip.so")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nano_hisparse import _hip

    _hip.load()  # fails loudly when the HIP library is missing
    return torch.device("cuda:0")


@pytest.fixture(params=["cpu", pytest.param("cuda:0", marks=pytest.mark.gpu)])
def device(request):
    """Runs a host-logic test on CPU tensors (the C oracle computes the
    kernels, installed as the CPU kernel provider) and, marked gpu, on
    cuda:0 through libnhs_hip.so."""
    import torch

    torch.set_num_threads(1)
    if request.param == "cpu":
        import cpu_provider

        cpu_provider.install()
        yield "cpu"
        cpu_provider.uninstall()
        return
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nano_hisparse import _hip

    _hip.load()
    yield request.param


@pytest.fixture
def cpu_kernels():
    """The oracle as CPU kernel provider, for CPU-only host-logic tests."""
    import cpu_provider

    cpu_provider.install()
    yield
    cpu_provider.uninstall()
