"""Build libmhc_hip.so (gfx950) in-tree with hipcc.

    python -m mhc_ascend_amd.csrc.build [--jobs N] [--verbose]

Each .hip translation unit is compiled to an object in parallel, then all
are linked into ``mhc_ascend_amd/libmhc_hip.so``; the same sources with
MHC_KERNEL_TIMING make ``libmhc_hip_timed.so``, the benchmark's build with
per-kernel HIP-event timing (include/mhc_hip_timing.h).  Alongside, g++ builds
``mhc_ascend_amd/_mhc_autograd.so``, the C++ autograd nodes of the fused
layers (autograd.cpp, a torch extension that calls the library through the
addresses of its C-ABI entry points).  Every call rebuilds from scratch (the
build is the "does it compile" check); outputs go to the package directory
and ``mhc_ascend_amd/csrc/_build``.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

CSRC = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(CSRC)
REPO = os.path.dirname(PKG)
INCLUDE = os.path.join(REPO, "include")
BUILD_DIR = os.path.join(CSRC, "_build")
LIB_NAME = "libmhc_hip.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
TIMED_LIB_PATH = os.path.join(PKG, "libmhc_hip_timed.so")
AUTOGRAD_NAME = "_mhc_autograd"
AUTOGRAD_PATH = os.path.join(PKG, AUTOGRAD_NAME + ".so")

SOURCES = ["abi.hip", "compat.hip", "dynamic.hip", "generic.hip", "layer.hip", "ops.hip", "sinkhorn.hip", "wide.hip",
           "wrapper.hip", "wrapper_gen.hip"]

ARCH = os.environ.get("MHC_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-fp32 VALU forms are disabled for device code: the compiler
    # emits them from plain float code otherwise.  The host pass warns that
    # it does not know the feature; that is expected.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
    "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _autograd_cmd(out: str):
    """g++ line for the torch extension (the include and library paths of
    torch.utils.cpp_extension; HIP headers for ATen's HIP stream API)."""
    import sysconfig

    import torch.utils.cpp_extension as ce

    incs = ce.include_paths("cuda") + [sysconfig.get_paths()["include"], INCLUDE]
    libdir = ce.library_paths()[0]
    return (["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
             "-DTORCH_API_INCLUDE_EXTENSION_H", f"-DTORCH_EXTENSION_NAME={AUTOGRAD_NAME}"]
            + [f"-I{i}" for i in incs]
            + [os.path.join(CSRC, "autograd.cpp"), "-o", out, f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu",
               "-ltorch_python", "-lc10_hip", "-ltorch_hip"])


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Build the product library, its benchmark twin with per-kernel timing
    (the same sources with MHC_KERNEL_TIMING, libmhc_hip_timed.so; only
    bench.py's per-kernel pass loads it) and the autograd extension."""
    hipcc = _hipcc()
    variants = ((LIB_PATH, BUILD_DIR, []), (TIMED_LIB_PATH, os.path.join(BUILD_DIR, "timed"), ["-DMHC_KERNEL_TIMING"]))
    objs = {lib: [] for lib, _, _ in variants}
    cmds = []
    for lib, bdir, defs in variants:
        os.makedirs(bdir, exist_ok=True)
        for src in SOURCES:
            obj = os.path.join(bdir, os.path.splitext(src)[0] + ".o")
            objs[lib].append(obj)
            cmds.append([hipcc, *COMMON_FLAGS, *defs, "-c", os.path.join(CSRC, src), "-o", obj])
    ag_tmp = AUTOGRAD_PATH + ".tmp"
    cmds.append(_autograd_cmd(ag_tmp))
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    os.replace(ag_tmp, AUTOGRAD_PATH)
    for lib, _, _ in variants:
        tmp = lib + ".tmp"
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs[lib]], verbose)
        os.replace(tmp, lib)
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args(argv)
    path = build(a.jobs, a.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
