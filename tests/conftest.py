import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gguf-rs-cli_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as _o
    _o.load()
    return _o


@pytest.fixture(scope="session")
def gpu():
    """The HIP sampler module; requires a visible GPU."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import gs_sampler
    gs_sampler.load_library()
    return gs_sampler


@pytest.fixture(scope="session")
def torch():
    """torch with a visible GPU (GPU tests only)."""
    import torch as _t
    if not _t.cuda.is_available():
        pytest.skip("no GPU")
    return _t
