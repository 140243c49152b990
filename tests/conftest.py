import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


# A sanitized build of the library (tests/support/host_sanitize.py) in place
# of the shipped and test builds, for the sanitizer run of the host tests.
SANITIZED = os.environ.get("LH_SANITIZED_LIBRARY")
if SANITIZED:
    import lunelette_amd
    lunelette_amd.LIBRARY = lunelette_amd.TEST_LIBRARY = SANITIZED


def pytest_configure(config):
    # Temporary files (checkpoint containers) stay inside the repository tree.
    if not config.option.basetemp:
        config.option.basetemp = os.path.join(ROOT, ".pytest_tmp")
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def product():
    import lunelette_amd
    return lunelette_amd.lib()


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def gpu(product):
    if product.lh_device_count() < 1:
        pytest.skip("no HIP device visible")
    return product
