"""In-tree build of the xsimgs_amd native libraries.

* ``libxsimgs_hip.so`` -- the C-ABI (include/*.h) with every HIP kernel, compiled by
  hipcc for gfx950. Packed-FP32 instruction selection is disabled.
* ``_C*.so`` -- the torch extension that re-exports the reference's op names over the C-ABI.

Object files go to ``xsimgs_amd/_build``; the two shared libraries sit in the package directory
so that they travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("XSG_OFFLOAD_ARCH", "gfx950")

# the slowest translation units first, so that the parallel build ends soonest
HIP_SOURCES = ["eval3d_bwd_g7.hip", "eval3d_bwd_g6.hip", "eval3d_bwd_g5.hip", "eval3d_bwd_g4.hip",
               "eval3d_bwd_g3.hip", "eval3d_bwd_g2.hip", "eval3d_bwd_g1.hip", "eval3d_bwd_g0.hip",
               "eval3d_fwd.hip", "tiling.hip", "camera.hip", "sh.hip", "capi.hip", "eval3d_bwd.hip",
               "eval3d_capi.hip", "nodes.hip", "calibrate.hip"]
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result"]

LIB_NAME = "libxsimgs_hip.so"


def ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def lib_path() -> str:
    return os.path.join(PKG, LIB_NAME)


def ext_path() -> str:
    return os.path.join(PKG, "_C" + ext_suffix())


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _stale(obj: str, src: str) -> bool:
    """True when obj is missing or older than src or any header beside it."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    deps.append(os.path.join(ROOT, "include", "xsimgs_amd.h"))
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def build_hip(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> str:
    """Compile every HIP source (only the stale ones when incremental) and link the library."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        if incremental and not _stale(obj, os.path.join(CSRC, src)):
            return obj
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose:
            print("  built", src, flush=True)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = lib_path() + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, lib_path())
    return lib_path()


def build_ext(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension as ce

    inc = ce.include_paths() + [sysconfig.get_paths()["include"], os.path.join(ROCM, "include")]
    libdirs = ce.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", os.path.join(CSRC, "torch_ext.cpp"),
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-fvisibility=hidden"]
    cmd += [f"-I{p}" for p in inc]
    cmd += [f"-L{p}" for p in libdirs] + [f"-Wl,-rpath,{p}" for p in libdirs]
    cmd += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-ltorch_hip",
            f"-L{PKG}", "-lxsimgs_hip", "-Wl,-rpath,$ORIGIN"]
    tmp = ext_path() + ".tmp"
    cmd += ["-o", tmp]
    _run(cmd)
    os.replace(tmp, ext_path())
    if verbose:
        print("  built torch extension", flush=True)
    return ext_path()


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def build_all(verbose: bool = False, incremental: bool = False) -> None:
    build_hip(verbose=verbose, incremental=incremental)
    build_ext(verbose=verbose)


if __name__ == "__main__":
    build_all(verbose=True, incremental="--incremental" in sys.argv)
    if "--oracle" in sys.argv:
        build_oracle()
