"""Shared fixtures and markers.

``gpu`` tests need a GPU and the built HIP library; everything else runs on
the CPU. The whole session uses a throwaway kernel cache (``AKO_CACHE_PATH``)
so tests never touch ``~/.ako``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from ako_amd.dispatcher.selector import reset_selector  # noqa: E402


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(autouse=True, scope="session")
def isolated_kernel_cache(tmp_path_factory):
    cache_dir = tmp_path_factory.mktemp("ako-cache")
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("AKO_CACHE_PATH", str(cache_dir / "kernel_cache.json"))
        reset_selector()
        yield
    reset_selector()
