"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

`hummingbird_amd._build.build_sanitized` compiles every source with both sanitizers on the host pass (the device
code is built as usual); this test builds that library and runs tests/test_abi.py against it in a child process
that preloads the clang sanitizer runtime, so every validator, overlap check and extent computation those tests
reach (fake-pointer layouts, the 400-layout brute force, the overflowing strides) runs instrumented. Any
sanitizer report aborts the child.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

from hummingbird_amd import _build

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(), reason="needs hipcc")
def test_abi_suite_is_clean_under_asan_and_ubsan():
    lib = _build.build_sanitized()
    env = dict(os.environ, HUMMINGBIRD_AMD_LIB=str(lib), LD_PRELOAD=str(_build.sanitizer_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", PYTHONPATH=str(ROOT))
    cmd = [sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi.py"), "-q", "-p", "no:cacheprovider",
           "-x", "-m", "not gpu"]
    res = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "Sanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert " passed" in out
    # the child really loaded the instrumented build (its validators trap, e.g., on signed overflow)
    probe = [sys.executable, "-c", "from hummingbird_amd import _lib; print(_lib.LIB_PATH); "
             "print(hex(_lib.load().hb_version is not None))"]
    res = subprocess.run(probe, cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and str(lib) in res.stdout, res.stdout + res.stderr
