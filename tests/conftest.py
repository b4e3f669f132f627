import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: longer CPU checks")


@pytest.fixture(scope="session")
def oracle():
    from oracle_libs import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_libs import Ref, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref was not built (the reference sources were absent)")
    return Ref()


@pytest.fixture(scope="session")
def gpu():
    import rustfox_amd
    g = rustfox_amd.Gpu(0)
    yield g
    g.close()
