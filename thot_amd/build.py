"""Builds libnott_hip.so (HIP kernels + C ABI) in-tree for gfx950.

Usage: python -m thot_amd.build   (or thot_amd.build.build_library()).
Objects go to thot_amd/_build/, the library to thot_amd/libnott_hip.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD = os.path.join(PKG_DIR, "_build")
LIB = os.path.join(PKG_DIR, "libnott_hip.so")
INCLUDE = os.path.join(REPO_DIR, "include")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM_LIB = "/opt/rocm/lib"

# Packed-fp32 VALU ops are disabled for every HIP translation unit.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build_library(jobs: int | None = None, verbose: bool = True) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs, "-Wl,-soname,libnott_hip.so",
           f"-L{ROCM_LIB}", f"-Wl,-rpath,{ROCM_LIB}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


HOST_SRC = os.path.join(PKG_DIR, "host", "nott_host.cpp")


def host_ext_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_nott_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_host(verbose: bool = True) -> str:
    """Builds the C++ host layer (include/nott_hip/host.hpp) as a Python
    extension with g++: host code only, every kernel lives in libnott_hip.so."""
    import sysconfig
    import torch
    tdir = os.path.dirname(torch.__file__)
    out = host_ext_path()
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           "-DTORCH_EXTENSION_NAME=_nott_host", "-D_GLIBCXX_USE_CXX11_ABI=1",
           f"-I{INCLUDE}", f"-I{tdir}/include", f"-I{tdir}/include/torch/csrc/api/include", "-I/opt/rocm/include",
           "-I" + sysconfig.get_paths()["include"], HOST_SRC, "-o", tmp,
           f"-L{PKG_DIR}", "-lnott_hip", f"-L{tdir}/lib", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_hip", "-ltorch_python", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tdir}/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host extension build failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    build_library()
    if "--lib-only" not in sys.argv:
        build_host()
