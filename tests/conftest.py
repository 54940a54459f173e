import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "boa-constrictor_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402,F401  (before any libboa_hip load: shared HIP runtime)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libboa_hip.so")
    config.addinivalue_line("markers", "slow: long-running")


def pytest_collection_modifyitems(config, items):
    # GPU tests run in the order the files define; nothing else to do
    pass


@pytest.fixture(scope="session")
def ora():
    from oracle import ora as _ora

    _ora.lib()
    return _ora


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from boa_amd import _native

    return _native.lib()
