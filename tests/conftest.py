"""Shared pytest setup: the `gpu` marker and import paths (repo root, oracle/)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ora():
    import oracle  # noqa: WPS433 (test-only import of the CPU oracle)

    oracle.lib()
    return oracle
