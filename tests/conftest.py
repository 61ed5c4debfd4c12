"""pytest configuration: markers, import paths, shared fixtures."""
import os
import sys

import pytest

TESTS = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(TESTS)
for p in (REPO, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle_bindings import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_bindings import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built (reference checkout not mounted)")
    return Ref()


@pytest.fixture(scope="session")
def tq4():
    import __graft_entry__
    return __graft_entry__.package()
