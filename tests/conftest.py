"""Shared pytest setup: the `gpu` marker, import paths and GPU fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


_gpu_count = None


def gpu_count() -> int:
    global _gpu_count
    if _gpu_count is None:
        from kvflux_amd import capi
        _gpu_count = capi.device_count()
    return _gpu_count


@pytest.fixture
def gpu():
    """Skips when no GPU is visible; returns device 0."""
    if gpu_count() == 0:
        pytest.skip("no GPU visible")
    from kvflux_amd import capi
    capi.call("kvflux_set_device", 0)
    return 0


@pytest.fixture(scope="session")
def v2():
    import kvflux_amd
    return kvflux_amd.v2
