import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "shannon-prime-burnhard_amd")
for p in (REPO, PKG, os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libspq4k.so")


@pytest.fixture(scope="session")
def oracle():
    from _oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from _oracle import Ref, ref_library_path
    if ref_library_path() is None:
        pytest.skip("oracle/_ref (the reference's ggml built from source) is not built")
    return Ref()


@pytest.fixture(scope="session")
def ctx():
    import spq4k
    c = spq4k.Context(0)
    yield c
    c.close()
