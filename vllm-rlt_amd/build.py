"""Build recipe of librlt_mi355x.so (gfx950) and its torch operators -- plain hipcc,
in-tree output.

Each .hip file is compiled to an object with hipcc for gfx950 only and the
objects are linked into ``librlt_mi355x.so`` next to this file (the C ABI, also
loaded with ctypes); ``csrc/torch_bindings.cpp`` is compiled against torch's
headers into ``_C.so``, which registers the ``torch.ops.rlt_mi355x`` operators
over that library.  Rebuilds every time it is called.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librlt_mi355x.so")
OPS_LIB = os.path.join(HERE, "_C.so")
SOURCES = ["paged_attention.hip", "spec_sampling.hip", "probabilities.hip", "kv_write.hip", "routing.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-const-variable",
    # no fused multiply-add contraction: the sampler's fp32 comparisons follow
    # torch-CPU arithmetic exactly
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(os.path.dirname(HERE), "include"),
]


def _compile(src):
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _torch_paths():
    """Include and library directories of the installed torch (no import of torch:
    its location is enough)."""
    import importlib.util

    root = os.path.dirname(importlib.util.find_spec("torch").origin)
    return ([os.path.join(root, "include"), os.path.join(root, "include", "torch", "csrc", "api",
                                                         "include")],
            os.path.join(root, "lib"))


def _bindings():
    """torch_bindings.cpp -> _C.so: the TORCH_LIBRARY(rlt_mi355x) operators, host code
    compiled by hipcc (no device code, no hipify), linked against librlt_mi355x.so."""
    incs, libdir = _torch_paths()
    src = os.path.join(CSRC, "torch_bindings.cpp")
    tmp = OPS_LIB + ".tmp"
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
           "-D_GLIBCXX_USE_CXX11_ABI=1", "-DUSE_ROCM=1",
           "-I", os.path.join(os.path.dirname(HERE), "include"), *sum((["-I", d] for d in incs), []),
           src, "-o", tmp, "-L", HERE, "-lrlt_mi355x", "-L", libdir, "-lc10", "-lc10_hip",
           "-ltorch_cpu", "-ltorch_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + libdir]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for torch_bindings.cpp:\n{proc.stderr[-4000:]}")
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


def build():
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], check=True)
    os.replace(tmp, LIB)
    _bindings()
    return LIB


if __name__ == "__main__":
    print(build())
