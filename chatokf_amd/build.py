"""Build the in-tree HIP library ``chatokf_amd/libokf_quant.so`` for gfx950.

Usage: ``python -m chatokf_amd.build`` (or ``__graft_entry__.build()``).
The library is compiled here, on the CPU, and travels to the GPU box as a
file; nothing is compiled at import time.

``python -m chatokf_amd.build --trace`` builds the diagnostic variant
``libokf_quant_trace.so`` (compiled with OKF_TRACE: the one-launch FFN
records per-workgroup phase timestamps, read by ``chatokf_amd/trace_ffn.py``).
"""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
# the C ABI (okf_quant.hip) and one translation unit per group of formats
# (okf_fmt_*.hip), compiled in parallel and linked into one library
SRCS = [os.path.join(CSRC, "okf_quant.hip")] + sorted(glob.glob(os.path.join(CSRC, "okf_fmt_*.hip")))
LIB = os.path.join(HERE, "libokf_quant.so")
OBJ = os.path.join(HERE, "_build")
LIB_TRACE = os.path.join(HERE, "libokf_quant_trace.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep private arrays in registers: LDS promotion of a prefetch buffer
    # serialises its loads
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)


def build(verbose: bool = False, trace: bool = False) -> str:
    obj_dir, lib = (OBJ + "_trace", LIB_TRACE) if trace else (OBJ, LIB)
    flags = FLAGS + (["-DOKF_TRACE"] if trace else [])
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o") for src in SRCS]
    jobs = min(len(SRCS), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([HIPCC, *flags, "-c", so[0], "-o", so[1]], verbose), zip(SRCS, objs)))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", lib + ".tmp"], verbose)
    os.replace(lib + ".tmp", lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True, trace="--trace" in sys.argv[1:]))
