"""pytest configuration: the `gpu` marker and shared fixtures.

CPU runs:  python -m pytest tests -m "not gpu"
GPU runs:  python -m pytest tests -m gpu   (on an MI355X box)
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        return np.load(os.path.join(REPO, "tests", "golden", name), allow_pickle=False)

    return load
