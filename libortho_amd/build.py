"""Builds libortho_amd/libortho_amd.so (the gfx950 HIP library behind the
C ABI of include/orth_hip.h) in-tree with hipcc.

    python -m libortho_amd.build          # or: python libortho_amd/build.py

Every .hip file under csrc/ is compiled for gfx950 only and linked into one
shared library.  No torch headers are involved there: the Python side binds
the plain C ABI with ctypes.  csrc/torch_ops.cpp, host code only, is then
compiled with g++ against torch's headers into the compiled binding
libortho_amd/_torch_ops*.so (the eager calls' fast path), linked to
libortho_amd.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libortho_amd.so")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # no packed FP32 arithmetic in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libortho_amd)")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def _stale(src: str, headers) -> bool:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(f) > t for f in [src, *headers])


def build(verbose: bool = False, changed_only: bool = False) -> str:
    """Compile every csrc/*.hip and link libortho_amd.so; returns its path.
    ``changed_only`` recompiles only sources newer than their objects (or
    than a header), for edit-compile loops."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    headers = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    headers.append(os.path.join(ROOT, "include", "orth_hip.h"))
    todo = [s for s in srcs if _stale(s, headers)] if changed_only else srcs
    jobs = min(max(1, len(todo)), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [os.path.join(BUILD, os.path.basename(s).replace(".hip", ".o")) for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def build_torch_ops(verbose: bool = False) -> str:
    """Compile csrc/torch_ops.cpp (host C++, torch extension) in-tree."""
    import sysconfig
    import torch
    import torch.utils.cpp_extension as ce
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(HERE, "_torch_ops" + suffix)
    src = os.path.join(CSRC, "torch_ops.cpp")
    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}",
                                                      "-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}"]
    libdirs = ce.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-w", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_torch_ops",
           "-DTORCH_API_INCLUDE_EXTENSION_H", *inc, src, "-o", out + ".tmp",
           *[f"-L{d}" for d in libdirs], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           f"-L{HERE}", "-l:libortho_amd.so", "-Wl,-rpath,$ORIGIN",
           *[f"-Wl,-rpath,{d}" for d in libdirs], "-L/opt/rocm/lib", "-lamdhip64"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch binding build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(out + ".tmp", out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    build(verbose=True, changed_only="--changed" in sys.argv)
    build_torch_ops(verbose=True)
    sys.exit(0)
