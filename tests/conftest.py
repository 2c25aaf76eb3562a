from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def product_lib():
    """The product library, built in-tree first if nothing is built yet."""
    from jeeves_amd import _lib, build

    if not _lib.LIB_PATH.exists():
        build.build(tests=True)
    return _lib.lib()


@pytest.fixture(scope="session")
def hooks_lib():
    """The GPU conformance-probe library (tests/csrc/testhooks.hip)."""
    from tests import helpers

    return helpers.hooks()
