import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import helpers
    return helpers.load_oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's own fh3_quant.c/fh3_ops.c build, when present."""
    import helpers
    lib = helpers.load_ref()
    if lib is None:
        pytest.skip("oracle/_ref/libfh3_ref.so not built (reference tree absent)")
    return lib


@pytest.fixture(scope="session")
def fh3():
    from fasth3inc_amd import fh3 as F
    F.lib()
    return F


@pytest.fixture(scope="session")
def gpu(fh3):
    """Initialised HIP module; fails (does not skip) when no gfx950 device."""
    fh3.init(int(os.environ.get("FH3_HIP_DEVICE", "0")))
    yield fh3
    fh3.set_path(fh3.PATH_AUTO)
