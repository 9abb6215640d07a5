"""The CPU checks of the C ABI (tests/test_capi.py) again, against the library
built with AddressSanitizer on its host code (``_build.build_sanitized_library``,
made by ``__graft_entry__.build()``).

They run in a child pytest with the sanitizer runtime preloaded (the Python
interpreter is not instrumented) and FRWKV_TEST_LIBRARY pointing the tests at
the sanitized build: argument checks, workspace sizing, the no-allocation
entry's size check and error reporting all execute under the sanitizer, which
aborts the child on the first invalid access. Leak checking is off: the HIP
runtime and PyTorch keep allocations until exit by design.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from flashrwkv_amd import _build

ROOT = Path(__file__).resolve().parents[1]


def test_c_abi_host_code_is_clean_under_address_sanitizer():
    runtime = _build.asan_runtime()
    if runtime is None:
        pytest.skip("no clang AddressSanitizer runtime under /opt/rocm/lib/llvm")
    if not _build.ASAN_LIB.exists():
        pytest.fail(f"{_build.ASAN_LIB} is not built; run __graft_entry__.build() "
                    "or _build.build_sanitized_library()")
    env = dict(os.environ)
    env["LD_PRELOAD"] = str(runtime)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1"
    env["FRWKV_TEST_LIBRARY"] = str(_build.ASAN_LIB)
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
         str(ROOT / "tests" / "test_capi.py")],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    report = proc.stdout[-3000:] + proc.stderr[-3000:]
    assert "AddressSanitizer" not in proc.stderr, report
    assert proc.returncode == 0, report
    assert " passed" in proc.stdout, report
