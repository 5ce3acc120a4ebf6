import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs the HIP path on an MI355X")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    if not os.path.exists(oracle_lib.ORACLE_SO):
        pytest.fail(f"{oracle_lib.ORACLE_SO} is missing: run __graft_entry__.build()")
    return oracle_lib.Oracle()


@pytest.fixture(scope="session")
def reference():
    import oracle_lib
    if not oracle_lib.have_reference():
        pytest.skip("oracle/_ref is built only where the reference sources are present")
    return oracle_lib.Reference()


@pytest.fixture(scope="session")
def nc():
    from nc_pkg import nc as pkg
    return pkg


@pytest.fixture(scope="session")
def gpu(nc):
    """The product library with the device initialised (GPU tests only)."""
    nc.init(0)
    return nc
