"""Shared test set-up: markers, import paths and the oracle libraries."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "hnsw-vector-db_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import load_oracle
    return load_oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle_lib import load_reference
    ref = load_reference()
    if ref is None:
        pytest.skip("oracle/_ref (the compiled reference) is not built here")
    return ref


@pytest.fixture(scope="session")
def ctx():
    import vdbg  # fails loudly when libvdbg.so is missing
    c = vdbg.Context(0)
    yield c
    c.close()
