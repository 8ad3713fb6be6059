"""Runs the host-only C-ABI tests of test_abi.py against a given libwkv build, in a
process that never imports torch (the sanitizer runtime is preloaded into it: see
test_abi_sanitized.py). Usage: python abi_sanitized_driver.py REPO_ROOT LIBRARY."""

import importlib.util
import inspect
import sys
import types
from pathlib import Path


def main() -> int:
    repo, lib = Path(sys.argv[1]), Path(sys.argv[2])
    sys.modules["torch"] = None  # importing it fails: the tests take the no-GPU branch
    spec = importlib.util.spec_from_file_location("wavelet_amd._lib", repo / "wavelet_amd" / "_lib.py")
    _lib = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(_lib)
    _lib.LIB_PATH = lib
    pkg = types.ModuleType("wavelet_amd")  # only _lib: the package proper imports torch
    pkg.__path__ = []
    pkg._lib = _lib
    sys.modules["wavelet_amd"] = pkg
    sys.modules["wavelet_amd._lib"] = _lib
    spec = importlib.util.spec_from_file_location("test_abi", repo / "tests" / "test_abi.py")
    tests = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(tests)
    ran = skipped = 0
    for name, fn in sorted(vars(tests).items()):
        if not name.startswith("test_") or not callable(fn) or inspect.signature(fn).parameters:
            continue
        try:
            fn()
        except ImportError as e:  # needs the torch-backed package
            skipped += 1
            print(f"skip {name}: {e}", flush=True)
            continue
        ran += 1
        print(f"ok {name}", flush=True)
    print(f"ran {ran} skipped {skipped}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
