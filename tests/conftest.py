"""Shared pytest setup: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs the oracle-vs-golden checks, host logic and the C-ABI
symbol checks on any machine; ``-m gpu`` runs the HIP parity tests and needs an
MI355X (gfx950) with the library built in-tree.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "turboquant-pro_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")
