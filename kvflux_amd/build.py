"""Build recipe of the native libraries (no cmake/ninja needed).

Produces, in-tree:
  kvflux_amd/lib/libkvflux_hip.so   gfx950 kernels + C ABI (include/kvflux_hip.h)
  kvflux_amd/lib/libkvflux.so       kvflux::v2 C++17 layer (g++, calls the C ABI)
  kvflux_amd/_kvflux<ext>.so        pybind11 binding of the C++ layer

Run `python -m kvflux_amd.build` (or __graft_entry__.build()). Every HIP
source is compiled for gfx950 only.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed FP32 VALU ops stay disabled on gfx950 (hipcc warns that the host
    # pass does not know the feature; that is harmless).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
    f"-I{INCLUDE}", f"-I{CSRC / 'hip'}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
             f"-I{INCLUDE}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd[:4])} ...")


def _compile_hip(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def build_hip(jobs: int = 8) -> Path:
    """Compiles every csrc/hip/*.hip for gfx950 and links libkvflux_hip.so."""
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    sources = sorted((CSRC / "hip").glob("*.hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile_hip, sources))
    out = LIB / "libkvflux_hip.so"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects),
          "-o", str(out)])
    return out


def build_host() -> Path:
    """Builds the kvflux::v2 C++ layer; it links only the C ABI library."""
    out = LIB / "libkvflux.so"
    sources = sorted((CSRC / "host").glob("*.cpp"))
    _run([CXX, *CXX_FLAGS, "-shared", *map(str, sources), f"-L{LIB}", "-lkvflux_hip",
          "-Wl,-rpath,$ORIGIN", "-o", str(out)])
    return out


def build_binding() -> Path:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / f"_kvflux{suffix}"
    py_include = sysconfig.get_paths()["include"]
    _run([CXX, *CXX_FLAGS, "-shared", f"-I{py_include}", f"-I{pybind11.get_include()}",
          "-fvisibility=hidden", str(CSRC / "bind" / "module.cpp"), f"-L{LIB}", "-lkvflux",
          "-lkvflux_hip", "-Wl,-rpath,$ORIGIN/lib", "-o", str(out)])
    return out


def build_all(jobs: int = 8) -> None:
    build_hip(jobs)
    build_host()
    build_binding()


if __name__ == "__main__":
    build_all()
    print("built", *sorted(p.name for p in LIB.glob("*.so")))
