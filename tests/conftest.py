import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O.Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import oracle as O
    if not os.path.exists(O.REF_PATH):
        pytest.skip("reference CPU build (oracle/_ref) not present")
    return O.Oracle(reference=True)
