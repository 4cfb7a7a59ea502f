"""Build recipe for libmars_amd.so (gfx950 only) and the CPU oracle.

``python mars_amd/build.py`` compiles every HIP / C++ source of the package
in-tree with hipcc for ``--offload-arch=gfx950``. It always recompiles.
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
BUILD = ROOT / "_build"
LIB = PKG / "libmars_amd.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"
# Packed-fp32 VALU ops stay disabled in every HIP compile (the host pass of
# hipcc ignores the feature with a warning).
NO_PK_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-std=c++17", "-O3", "-fPIC", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
SOURCES = ["api.hip", "kernels.hip", "batch.hip", "batch_mm.hip", "batch_rq.hip", "multi.hip", "insert.hip", "tiled.hip", "maintain.hip", "noalloc.hip", "scan8.hip", "scan8m.hip",
           "corpus.cpp", "formats.cpp", "nsn.cpp", "shim.cpp"]
DRIVER_SRC = ROOT / "tests" / "cpp" / "shim_driver.cpp"
DRIVER = ROOT / "tests" / "cpp" / "shim_driver"
ENGINE = PKG / "mars_engine"


def _compile(src: str) -> Path:
    out = BUILD / (src + ".o")
    path = CSRC / src
    if src.endswith(".hip"):
        cmd = [HIPCC, "-x", "hip", f"--offload-arch={ARCH}", *COMMON, *NO_PK_FP32, "-c", str(path), "-o", str(out)]
    else:
        # host-only C++: the system compiler (hipcc would compile .cpp as HIP)
        cmd = [CXX, *COMMON, "-march=x86-64-v3", "-Wall", "-Wextra", "-c", str(path), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return out


def build_library(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    # the C++ driver of the reference-API shim (tests run it)
    cmd = [CXX, "-std=c++17", "-O2", f"-I{ROOT / 'include'}", str(DRIVER_SRC), "-o", str(DRIVER),
           f"-L{PKG}", "-lmars_amd", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/../../mars_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"driver build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # the JSON-line engine server over the C ABI
    cmd = [CXX, "-std=c++17", "-O2", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", str(CSRC / "engine.cpp"), "-o",
           str(ENGINE), f"-L{PKG}", "-lmars_amd", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"engine build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {LIB}, {DRIVER} and {ENGINE}")
    return LIB


def build_oracle(verbose: bool = False) -> None:
    """Compile the CPU oracle (and oracle/_ref when the reference tree is present)."""
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    r = subprocess.run([make, "-B", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(r.stdout.strip())


if __name__ == "__main__":
    build_library(verbose=True)
    if "--no-oracle" not in sys.argv:
        build_oracle(verbose=True)
