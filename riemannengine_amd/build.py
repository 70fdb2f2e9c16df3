"""Build the native parts of riemannengine_amd in-tree.

* ``libriemann_hip.so`` — the gfx950 HIP kernels behind the C ABI declared in
  ``include/riemann_hip.h`` (hipcc, one object per translation unit).
* ``_C*.so`` — the C++ host layer (CoordinateManager / SparseTensor /
  RiemannConvolution over LibTorch) and its pybind11 module, compiled with
  g++ against the installed torch and linked to ``libriemann_hip.so``.

Run ``python -m riemannengine_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(CSRC, "host")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
HIP_LIB = os.path.join(PKG, "libriemann_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_SOURCES = ["abi.hip", "sort.hip", "hash.hip", "kmap.hip", "conv.hip", "pool.hip", "norm.hip"]
# gfx950 only. Packed-FP32 instructions are disabled: the compiler would
# otherwise form v_pk_* FP32 ops from plain float code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE, "-I" + CSRC,
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip(jobs: int = 4) -> str:
    """Compile the HIP kernels and link libriemann_hip.so; returns its path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    objs = []

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libriemann_hip.so"])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def _torch_paths():
    import torch  # noqa: F401  (only for its install location)
    from torch.utils import cpp_extension as ce
    tdir = os.path.dirname(os.path.abspath(__import__("torch").__file__))
    incs = ce.include_paths()
    libdir = os.path.join(tdir, "lib")
    return incs, libdir


def build_host() -> str:
    """Compile the C++ host layer + pybind11 module (_C) against LibTorch."""
    incs, libdir = _torch_paths()
    import torch
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(PKG, "_C" + suffix)
    srcs = sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp"))
    os.makedirs(BUILD, exist_ok=True)
    cxx = shutil.which("g++") or "g++"
    common = ["-O2", "-std=c++17", "-fPIC", "-DTORCH_EXTENSION_NAME=_C",
              "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              "-I" + INCLUDE, "-I" + HOST, "-I" + os.path.join(ROCM, "include"),
              "-I" + sysconfig.get_paths()["include"]]
    for i in incs:
        common += ["-isystem", i]
    objs = []

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD, "host_" + os.path.basename(src).replace(".cpp", ".o"))
        _run([cxx, *common, "-c", src, "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = out + ".tmp"
    _run([cxx, "-shared", "-o", tmp, *objs,
          "-L" + libdir, "-Wl,-rpath," + libdir,
          "-L" + PKG, "-Wl,-rpath,$ORIGIN", "-lriemann_hip",
          "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
          "-L" + os.path.join(ROCM, "lib"), "-lamdhip64"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_hip()
    if os.path.isdir(HOST) and any(f.endswith(".cpp") for f in os.listdir(HOST)):
        build_host()


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    {"hip": build_hip, "host": build_host, "all": build_all}[what]()
    print("built", what)
