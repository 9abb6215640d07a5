"""Shared pytest configuration: the `gpu` marker and repo-root imports."""

from __future__ import annotations

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built native library")
    # FRWKV_TEST_LIBRARY: run the C-ABI tests against another build of the
    # library (the host-sanitized one, tests/test_capi_asan.py).
    other = os.environ.get("FRWKV_TEST_LIBRARY")
    if other:
        from flashrwkv_amd import capi

        capi.LIBRARY = Path(other)
