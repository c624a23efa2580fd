"""Shared pytest setup: the `gpu` marker, repo-root imports, oracle build."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and librqf_hip.so")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    yield
