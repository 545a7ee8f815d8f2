"""Builds ``libastra_market.so`` (the HIP engine + C ABI) in-tree for gfx950.

Sources: ``csrc/market.hip`` (the VecMarket engine, include/astra_market.h) and
``csrc/high_low.hip`` (the high-low game's move kernels, include/astra_high_low.h).

Usage: ``python astra-cuda_amd/astra_cuda/build.py`` or ``astra_cuda.build.build()``.
The library links the HIP runtime by its SONAME (libamdhip64.so.7); imported after
torch, it binds to the runtime torch already loaded, so both share streams.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(PKG_DIR))
CSRC = os.path.join(os.path.dirname(PKG_DIR), "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libastra_market.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = [os.path.join(CSRC, "market.hip"), os.path.join(CSRC, "high_low.hip")]

ARCH = os.environ.get("ASTRA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    # keep the compiler from emitting packed FP32 ops (unused here anyway)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP engine cannot be built")


BINDING_SRC = os.path.join(CSRC, "bindings.cpp")


def binding_path() -> str:
    import sysconfig
    return os.path.join(PKG_DIR, "_C" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_binding(verbose: bool = False) -> str:
    """Compile the pybind11 module astra_cuda._C (csrc/bindings.cpp, the reference's
    market_bindings.cc surface over the C ABI) against torch's headers and libraries,
    linked to libastra_market.so in the same directory. Always recompiles."""
    import sysconfig
    import torch
    tdir = os.path.dirname(torch.__file__)
    incs = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
            "/opt/rocm/include", sysconfig.get_paths()["include"], INCLUDE]
    out = binding_path()
    tmp = out + ".tmp"
    cxx = os.environ.get("CXX", "g++")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *(f"-I{d}" for d in incs), BINDING_SRC,
           f"-L{os.path.join(tdir, 'lib')}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python", f"-L{PKG_DIR}", "-l:" + LIB_NAME,
           # the engine library next to the module, and torch's libraries
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(tdir, 'lib')}", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cxx} failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> str:
    """Compile the sources into the package directory. Always recompiles."""
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", *SOURCES, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_binding(verbose="-v" in sys.argv))
