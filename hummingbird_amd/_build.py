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


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
