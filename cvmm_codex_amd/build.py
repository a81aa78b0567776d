"""Build libcvmm_hip.so (gfx950) and the host glue module in-tree.

Each ``csrc/*.hip`` file compiles to an object with hipcc, in parallel with
the host glue (``csrc/host/cvmm_host.cpp``, g++ against torch's headers); one
link step produces ``cvmm_codex_amd/libcvmm_hip.so`` and a second links the
glue into ``cvmm_codex_amd/_host*.so`` against it.  Run ``python -m
cvmm_codex_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcvmm_hip.so")
ARCH = os.environ.get("CVMM_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-munsafe-fp-atomics",
    # packed fp32 VALU ops stay off: plain float code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


HOST_SRC = os.path.join(CSRC, "host", "cvmm_host.cpp")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
HOST_NAME = "_host"


def _host_flags():
    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    cflags = ["-O2", "-std=c++17", "-fPIC", f"-DTORCH_EXTENSION_NAME={HOST_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
              f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-I" + INCLUDE,
              "-I" + sysconfig.get_paths()["include"], *["-I" + p for p in include_paths()],
              # torch's current HIP stream (c10/hip/HIPStream.h) for the C++ autograd function
              "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "include")]
    ldflags = [*["-L" + p for p in library_paths()], *["-Wl,-rpath," + p for p in library_paths()],
               "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-L" + HERE, "-lcvmm_hip",
               "-Wl,-rpath,$ORIGIN"]
    return cflags, ldflags, sysconfig.get_config_var("EXT_SUFFIX")


def _compile_host(cflags) -> str:
    obj = os.path.join(BUILD, "cvmm_host.o")
    r = subprocess.run(["g++", *cflags, "-c", HOST_SRC, "-o", obj], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for {HOST_SRC}:\n{r.stderr}")
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs) + 1, max(1, (os.cpu_count() or 4)), 16)
    cflags, ldflags, ext_suffix = _host_flags()
    with cf.ThreadPoolExecutor(jobs) as ex:
        host_obj = ex.submit(_compile_host, cflags)
        objs = list(ex.map(_compile, srcs))
        host_obj = host_obj.result()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libcvmm_hip.so", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    host = os.path.join(HERE, HOST_NAME + ext_suffix)
    r = subprocess.run(["g++", "-shared", host_obj, "-o", host + ".tmp", *ldflags], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host glue link failed:\n{r.stderr}")
    os.replace(host + ".tmp", host)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources and {host}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
