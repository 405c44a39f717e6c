import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libaffx.so")


def pytest_collection_modifyitems(config, items):
    # GPU tests run in file order; nothing else to do
    return


@pytest.fixture(scope="session")
def orc():
    from oracle import build, load_oracle
    from oracle.binding import ORACLE_SO
    if not os.path.exists(ORACLE_SO):
        build(ref=False)
    return load_oracle()


@pytest.fixture(scope="session")
def c1_codebook():
    return np.fromfile(os.path.join(GOLDEN, "c1_codebook.bin"), dtype="<u4")


@pytest.fixture(scope="session")
def small():
    return np.load(os.path.join(GOLDEN, "small.npz"))


@pytest.fixture(scope="session")
def scalars():
    return np.load(os.path.join(GOLDEN, "scalars.npz"))
