"""Shared test setup: import paths, the `gpu` marker, library fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "flash-trie_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


def _ensure_built():
    import build as ftbuild  # flash-trie_amd/build.py
    if not ftbuild.built():
        ftbuild.build()


@pytest.fixture(scope="session")
def ft():
    """The product module `flashtrie` (HIP library behind it)."""
    _ensure_built()
    import flashtrie
    return flashtrie


@pytest.fixture(scope="session")
def po():
    """The CPU parity oracle (test infrastructure)."""
    import pyoracle
    pyoracle.lib()
    return pyoracle
