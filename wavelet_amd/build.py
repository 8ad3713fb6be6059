"""Builds libwkv.so (the C-ABI HIP library) in-tree for gfx950.

    python -m wavelet_amd.build

hipcc compiles every ``csrc/*.hip`` source to an object and links them into
``wavelet_amd/libwkv.so``. The library links only the HIP runtime: no torch
symbols cross the C ABI, so the same file is what a ctypes / cgo / JNI binding
would load.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libwkv.so"
PHASE_LIB = PKG / "libwkv_phase.so"  # profiling build (build_phase_clocks)
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Code object v5: loadable by the HIP runtime torch bundles as well as /opt/rocm's.
    "-mcode-object-version=5",
    # Packed fp32 VALU ops are kept off for the whole device build.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-source additions.
#   decode_gqa.hip, prefill_gqa.hip: MFMA accumulators in ordinary VGPRs. Its online softmax
#   rescales the output accumulators in place; with the accumulators in AGPRs
#   the compiler copies all of them to VGPRs and back on every tile (64 moves
#   per tile, measured in the ISA), whether or not a rescale happens. Its
#   kernels need at most ~200 registers, so nothing is lost. (decode_mla.hip
#   keeps AGPRs: its 1-wave-per-SIMD kernels use more than 256 registers.)
#   sampler.hip: no machine sinking. Its passes issue the loads of several
#   row chunks before using the first; the sinking pass moves each load back
#   down to its first use (into the branches that follow), leaving one load
#   in flight per thread (measured in the ISA: 4 batched loads in the max
#   pass only; the sampler 4% slower).
EXTRA_FLAGS = {
    "decode_gqa.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "prefill_gqa.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],  # the same tile code
    "sampler.hip": ["-mllvm", "-disable-machine-sink"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


# Host-code sanitizers for a CPU-only check of the C ABI's host side (argument
# validation, plans, sizes): every -fsanitize= applies to the host compilation
# only (-Xarch_host); the device code is built as usual. The library links the
# shared sanitizer runtime, which the process that loads it preloads
# (asan_runtime()).
SANITIZE_COMPILE = [
    "-Xarch_host", "-g",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
]
SANITIZE_LINK = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-shared-libsan"]


def _build(out: Path, compile_extra: list[str], link_extra: list[str], verbose: bool) -> Path:
    cc = hipcc()
    inc = ["-I", str(PKG.parent / "include")]
    with tempfile.TemporaryDirectory(prefix="wkv_build_") as tmpdir:
        objs = []
        cmds = []
        for src in sources():
            obj = Path(tmpdir) / (src.stem + ".o")
            objs.append(obj)
            cmds.append([cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), *compile_extra, *inc, "-c", str(src),
                         "-o", str(obj)])
        with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = out.with_suffix(".so.tmp")
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link_extra, *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile every source (one object each, in parallel) and link libwkv.so (always rebuilds)."""
    return _build(LIB, [], [], verbose)


def build_phase_clocks(out: Path | None = None, verbose: bool = False) -> Path:
    """The library with the MLA decode's per-phase cycle stamps (WKV_PHASE_CLOCKS;
    read by `bench.py --phase-clocks`), at `out` (default PHASE_LIB). Profiling only."""
    return _build(Path(out) if out is not None else PHASE_LIB, ["-DWKV_PHASE_CLOCKS"], [], verbose)


def build_sanitized(out: Path, verbose: bool = False) -> Path:
    """The same library with AddressSanitizer and UndefinedBehaviorSanitizer on its host code, at `out`."""
    return _build(Path(out), SANITIZE_COMPILE, SANITIZE_LINK, verbose)


def asan_runtime() -> Path | None:
    """The shared AddressSanitizer runtime of the compiler that builds the library (None if absent)."""
    clang = Path(hipcc()).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path(hipcc()).resolve().parent.parent / "llvm" / "bin" / "clang"
    if not clang.exists():
        return None
    proc = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = Path(proc.stdout.strip())
    return path if proc.returncode == 0 and path.is_absolute() and path.exists() else None


if __name__ == "__main__":
    if "--phase-clocks" in sys.argv[1:]:
        print(build_phase_clocks(verbose=True))
    else:
        print(build(verbose=True))
