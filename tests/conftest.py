import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")
    config.addinivalue_line("markers", "slow: long CPU test")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class ClfEnv:
    """Sets or clears CLF_* path switches for one test and makes the library
    re-read them (it reads them once per process otherwise)."""

    def __init__(self, mp):
        self._mp = mp

    def setenv(self, name, value):
        from cliffordcuda_amd import _lib
        self._mp.setenv(name, value)
        _lib.reload_options()

    def delenv(self, name, raising=True):
        from cliffordcuda_amd import _lib
        self._mp.delenv(name, raising=raising)
        _lib.reload_options()


@pytest.fixture
def clf_env(monkeypatch):
    env = ClfEnv(monkeypatch)
    yield env
    monkeypatch.undo()
    from cliffordcuda_amd import _lib
    if _lib._lib is not None:
        _lib.reload_options()

