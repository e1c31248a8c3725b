import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libwsl.so")


def has_gpu() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    if not has_gpu():
        pytest.skip("no GPU")
    import torch
    return torch.device("cuda:0")


@pytest.fixture
def wsl_opts():
    """Sets libwsl's path overrides for one test, by name (``_native.OPTIONS``:
    ``wsl_opts(decode_passes=-1)``), and restores every override when the test ends."""
    from weightshared_torchtitan_amd import _native
    saved = {k: _native.get_option(k) for k in _native.OPTIONS}

    def set_opts(**kw):
        for k, v in kw.items():
            _native.set_option(k, v)

    yield set_opts
    for k, v in saved.items():
        _native.set_option(k, v)
