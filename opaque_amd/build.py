"""Builds ``libopaque_dp.so`` (HIP kernels + C ABI) in-tree for gfx950.

Usage: ``python -m opaque_amd.build`` (or ``__graft_entry__.build()``).
The library is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libopaque_dp.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["odp_abi.hip", "odp_lora.hip", "odp_clip.hip", "odp_noise.hip", "odp_linear.hip", "odp_moments.hip",
           "odp_calib.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed-FP32 instructions are kept out of generated code on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build opaque_amd")


def build(verbose: bool = False) -> Path:
    """Compile every kernel source into one shared library. Always recompiles."""
    srcs = [str(CSRC / s) for s in SOURCES if (CSRC / s).exists()]
    tmp = LIB_PATH.with_name(LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc_path(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *srcs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        noise = [
            ln
            for ln in proc.stderr.splitlines()
            if "packed-fp32-ops" not in ln and ln.strip()
        ]
        if noise:
            print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


SAN_DIR = PKG_DIR / "_asan_build"
SAN_LIB = SAN_DIR / LIB_NAME
# The host side of the library instrumented for address and undefined-
# behaviour errors (device code is built as usual).  It is loaded only by
# the CPU test of the C ABI's argument and error handling, in a process
# that preloads the sanitizer runtime.
SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-Xarch_host", "-fsanitize=address",
             "-Xarch_host", "-fsanitize=undefined"]


def sanitizer_runtime() -> Path | None:
    """The compiler's AddressSanitizer runtime, which a process must preload
    to load the instrumented library."""
    llvm = Path(hipcc_path()).resolve().parent.parent / "llvm"
    for cand in sorted(llvm.glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")) + \
            sorted(Path("/opt/rocm/llvm").glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")):
        return cand
    return None


def build_sanitized(verbose: bool = False) -> Path:
    """Compile opaque_amd/_asan_build/libopaque_dp.so with the sanitizers on
    the host code; skipped when it is newer than every source."""
    srcs = [CSRC / s for s in SOURCES] + sorted(CSRC.glob("*.h")) + [INCLUDE / "opaque_dp.h"]
    if SAN_LIB.exists() and SAN_LIB.stat().st_mtime > max(p.stat().st_mtime for p in srcs):
        return SAN_LIB
    SAN_DIR.mkdir(exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-O3"] + SAN_FLAGS
    tmp = SAN_LIB.with_name(LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc_path(), *flags, f"-I{INCLUDE}", f"-I{CSRC}", *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc (sanitized) failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, SAN_LIB)
    return SAN_LIB


HOST_SRC = CSRC / "odp_host.cpp"
HOST_DIR = PKG_DIR / "_host_build"
HOST_NAME = "_odp_host"


def build_host(verbose: bool = False) -> Path:
    """Compile the host-side helper (a torch C++ extension, no device code)
    into opaque_amd/_host_build/_odp_host.so.  Always recompiles."""
    import torch.utils.cpp_extension as ext

    HOST_DIR.mkdir(exist_ok=True)
    for stale in HOST_DIR.glob("*"):
        if stale.is_file():
            stale.unlink()
    ext.load(name=HOST_NAME, sources=[str(HOST_SRC)], build_directory=str(HOST_DIR),
             extra_cflags=["-O2"], verbose=verbose)
    return HOST_DIR / f"{HOST_NAME}.so"


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_host(verbose=True))
