"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

libwkv is rebuilt with -fsanitize=address,undefined on its host code only (the
device code as usual) and loaded into a fresh process with the sanitizer
runtime preloaded; that process runs every host-only test of test_abi.py
(argument validation, launch plans, workspace sizes, error strings) and halts on
the first report. Host-only: the tests hand the library fake device pointers, so
this runs only where no GPU is visible."""

import os
import re
import subprocess
import sys
from pathlib import Path

import pytest

from wavelet_amd import build
from test_abi import _no_gpu

ROOT = Path(__file__).resolve().parents[1]


def _toolchain() -> bool:
    try:
        build.hipcc()
    except RuntimeError:
        return False
    return build.asan_runtime() is not None


pytestmark = [
    pytest.mark.skipif(not _no_gpu(), reason="fake device pointers: host-only test"),
    pytest.mark.skipif(not _toolchain(), reason="hipcc or its AddressSanitizer runtime is missing"),
]


def test_host_code_under_asan_and_ubsan(tmp_path):
    lib = build.build_sanitized(tmp_path / "libwkv_san.so")
    env = dict(os.environ,
               LD_PRELOAD=str(build.asan_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",  # the interpreter's own allocations are not leaks
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([sys.executable, str(ROOT / "tests" / "abi_sanitized_driver.py"), str(ROOT), str(lib)],
                          env=env, capture_output=True, text=True, timeout=600)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-6000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    ran = int(re.search(r"ran (\d+) skipped", out).group(1))
    assert ran >= 10, out
