"""Builds `libhummingbird_amd.so` (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Each source is compiled to an object in parallel, then linked. The shared library lands next to this file,
where `hummingbird_amd._lib` loads it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libhummingbird_amd.so"
ARCH = "gfx950"
SOURCES = ("api.cpp", "cross.cpp", "dense.hip", "band.hip", "band_ring.hip", "band_tiled.hip", "fp32.hip", "elementwise.hip",
           "proj.hip", "dit_block.hip")

# Device flags. Packed fp32 instructions are disabled for every HIP source: hipcc -O3 would otherwise form
# v_pk_{add,mul,fma}_f32 from ordinary float code. Floating-point contraction is off so that separately
# written products and sums keep their own roundings (the reference's cast points, and exact cancellation of
# identical differential branches); every fused multiply-add in the kernels is an explicit __fmaf_rn.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-ffp-contract=off"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"--offload-arch={ARCH}", f"-I{ROOT / 'include'}"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build hummingbird_amd")
    return path


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *COMMON_FLAGS]
    if src.suffix == ".hip":
        cmd += DEVICE_FLAGS
    cmd += ["-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link the shared library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        list(pool.map(lambda so: _compile(CSRC / so[0], so[1], verbose), zip(SOURCES, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB)
    return LIB


# Host-side sanitizer build (CPU checks of the C ABI's validators): every source's host pass gets AddressSanitizer
# and UndefinedBehaviorSanitizer; the device code is built as usual. The library is linked without the sanitizer
# runtime, which the process that loads it preloads (sanitizer_runtime()).
SAN_DIR = PKG / "_build_san"
SAN_LIB = SAN_DIR / "libhummingbird_amd.so"
SANITIZE_HOST_FLAGS = ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
                       "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer -Xarch_host -g").split()


def sanitizer_runtime() -> Path:
    """The clang AddressSanitizer runtime (which carries the UndefinedBehaviorSanitizer handlers) of hipcc."""
    root = Path(hipcc()).resolve().parent.parent / "lib" / "llvm" / "lib" / "clang"
    if not root.exists():
        root = Path("/opt/rocm/lib/llvm/lib/clang")
    found = sorted(root.glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError(f"no libclang_rt.asan-x86_64.so under {root}")
    return found[-1]


def build_sanitized(verbose: bool = False) -> Path:
    """Compile every source with the host sanitizers and link `_build_san/libhummingbird_amd.so`."""
    SAN_DIR.mkdir(exist_ok=True)
    objs = [SAN_DIR / (Path(s).stem + ".o") for s in SOURCES]

    def comp(src: Path, obj: Path) -> None:
        cmd = [hipcc(), *COMMON_FLAGS, *SANITIZE_HOST_FLAGS] + (DEVICE_FLAGS if src.suffix == ".hip" else [])
        cmd += ["-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc (sanitized host) failed on {src.name}:\n" + res.stderr[-4000:])

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        list(pool.map(lambda so: comp(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(SAN_LIB)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("sanitized link failed:\n" + res.stdout + res.stderr)
    return SAN_LIB


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
