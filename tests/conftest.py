"""Shared test setup: import paths, the `gpu` marker, the built HIP library."""

from __future__ import annotations

from pathlib import Path
import sys

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
PACKAGE_ROOT = REPO_ROOT / "rdna3-fastmm_amd"
for path in (str(REPO_ROOT), str(PACKAGE_ROOT)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")
    from rdna3_fastmm._build import LIBRARY_PATH, build_library

    if not LIBRARY_PATH.exists():
        build_library()
