"""Build libmoe_route.so (gfx950) in-tree with hipcc.

Usage: python -m moe_route.build   (or moe_route.build.build()).
The library lands next to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
CSRC = os.path.join(PKG_ROOT, "csrc")
REPO = os.path.dirname(PKG_ROOT)
LIB_NAME = "libmoe_route.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SOURCES = ["router_gemm.hip", "topk.hip", "route_fused.hip", "route_small.hip", "dispatch.hip",
           "permute.hip", "combine.hip", "grouped_gemm.hip", "quant_i8.hip", "moe_capi.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
# A C++ host program that uses the library through its C ABI only (no torch).
EXAMPLE_SRC = os.path.join(PKG_ROOT, "examples", "moe_step.cpp")
EXAMPLE_BIN = os.path.join(HERE, "moe_step")

FLAGS = [
    "-O3", "-std=c++20", "-fPIC", "-shared",
    "--offload-arch=gfx950",
    # packed fp32 VALU ops are kept out of every device function
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(proc, what):
    out, _ = proc.communicate()
    out = "\n".join(l for l in out.splitlines()
                    if "packed-fp32-ops" not in l)  # host pass does not know the feature
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed on %s (%d):\n%s" % (what, proc.returncode, out))
    return out


def build(verbose: bool = False) -> str:
    """Compile every HIP source of the library (in parallel), link the .so;
    returns its path."""
    objdir = os.path.join(HERE, "_obj")
    os.makedirs(objdir, exist_ok=True)
    inc = ["-I", os.path.join(REPO, "include"), "-I", CSRC]
    compile_flags = [f for f in FLAGS if f != "-shared"]
    procs, objs = [], []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        # .cpp sources also hold HIP host code
        cmd = [HIPCC] + compile_flags + inc + ["-x", "hip", "-c", os.path.join(CSRC, src),
                                               "-o", obj]
        procs.append((_run(cmd, verbose), src))
    logs = [_finish(p, src) for p, src in procs]
    tmp = LIB_PATH + ".tmp"
    link = _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950"] + objs + ["-o", tmp], verbose)
    logs.append(_finish(link, "link"))
    if verbose:
        for l in logs:
            if l.strip():
                print(l)
    os.replace(tmp, LIB_PATH)
    # host-only example against the installed library (rpath: next to the .so)
    ex = _run(["g++", "-O2", "-std=c++17", EXAMPLE_SRC, "-I", os.path.join(REPO, "include"),
               "-I", os.path.join(ROCM, "include"), "-D__HIP_PLATFORM_AMD__",
               "-L", HERE, "-lmoe_route", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
               "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
               "-o", EXAMPLE_BIN], verbose)
    _finish(ex, "examples/moe_step.cpp")
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
