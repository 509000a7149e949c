"""Shared pytest setup: the `gpu` marker, repo-root imports and the engine fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def backend():
    """The engine on cuda:0. GPU tests fail (not skip) when no gfx950 device is usable,
    like the reference's explicitly enabled GPU suites (CudaTensorTest.java:11-13)."""
    from jax4j_amd import Mi355xBackend

    be = Mi355xBackend()
    assert be.is_available(), "MI355X (gfx950) explicitly required for -m gpu tests"
    info = be.device_info()
    assert info["arch"].startswith("gfx950"), info
    return be
