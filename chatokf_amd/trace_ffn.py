"""Per-phase timestamps of the one-launch FFN (ffn_mfma_kernel at the Bonsai
shape, ffn_fused_kernel otherwise) on a GPU.

Usage (after ``python -m chatokf_amd.build --trace``)::

    python chatokf_amd/trace_ffn.py [--launches 64]

(as a file, not with -m: the package must not be imported before the
library path is set)

Loads the diagnostic library ``libokf_quant_trace.so`` (built with
OKF_TRACE: every workgroup records s_memrealtime, a 100 MHz device counter,
at seven points of each launch), runs the benchmark's FFN step (Q2_0 gate /
up 6144 x 2048 with the SiLU, down 2048 x 6144, weights rotated over >= 1 GiB
of copies like bench.py) back to back, once with each one-launch kernel,
and prints a markdown summary per kernel: per phase the median over
launches of the workgroups' minimum, median and maximum time, and per
launch its span and the gap to the next launch.
"""
import argparse
import ctypes
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if "chatokf_amd" in sys.modules:
    raise SystemExit("run this file directly (python chatokf_amd/trace_ffn.py), not with -m")
# (--lib PATH: another build with OKF_TRACE; read here, before the import)
_lib = sys.argv[sys.argv.index("--lib") + 1] if "--lib" in sys.argv else os.path.join(HERE, "libokf_quant_trace.so")
os.environ["OKF_LIB"] = os.path.abspath(_lib)
sys.path.insert(0, os.path.dirname(HERE))

import torch  # noqa: E402

import chatokf_amd as ok  # noqa: E402
from chatokf_amd import synth  # noqa: E402

NP, WG, L = 8, 256, 64  # points a workgroup (7 the epoch), workgroups, ring slots (okf_ffn.h)
PHASES = [
    ("issue", 0, 1, "start -> every weight / x load issued (wavefront 0)"),
    ("x", 1, 2, "-> x arrived and staged as digit planes"),
    ("phase A", 2, 3, "-> gate / up rows done, g written (last wavefront)"),
    ("barrier", 3, 4, "-> grid barrier released"),
    ("g", 4, 5, "-> g read back and staged"),
    ("phase B", 5, 6, "-> down rows done (last wavefront)"),
]


def trace(enc, refs, ptrs, n):
    """Runs n okf_ffn calls back to back on enc after a warm-up; returns the
    markdown rows of the phase table and the wall time a call."""
    lib = enc._lib
    lib.okf_ffn_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    ffn = lib.okf_ffn

    def step(i):
        gr, ur, dr = refs[i % len(refs)]
        if ffn(enc.h, gr, ur, dr, *ptrs):
            raise RuntimeError("okf_ffn failed")

    for i in range(200):
        step(i)
    enc.sync()
    t0 = time.perf_counter()
    for i in range(n):
        step(200 + i)
    enc.sync()
    wall = (time.perf_counter() - t0) / n
    buf = np.zeros(L * WG * NP, dtype=np.uint64)
    if lib.okf_ffn_trace_read(buf.ctypes.data, buf.size):
        raise RuntimeError("okf_ffn_trace_read failed")
    t = buf.reshape(L, WG, NP).astype(np.int64)
    ep = t[:, 0, 7]
    last = int(ep.max())
    want = set(range(last - n + 1, last + 1))
    runs = sorted((int(ep[s]), s) for s in range(L) if int(ep[s]) in want and (t[s, :, 7] == ep[s]).all())
    us = 0.01  # one tick of the 100 MHz counter
    rows = {name: [] for name, *_ in PHASES}
    spans, gaps, starts = [], [], []
    for j, (e, s) in enumerate(runs):
        tt = t[s, :, :7]
        start = tt[:, 0].min()
        starts.append((tt[:, 0].max() - start) * us)
        for name, a, b, _ in PHASES:
            d = (tt[:, b] - tt[:, a]) * us
            rows[name].append((d.min(), np.median(d), d.max()))
        spans.append((tt[:, 6].max() - start) * us)
        if j + 1 < len(runs) and runs[j + 1][0] == e + 1:
            gaps.append((t[runs[j + 1][1], :, 0].min() - tt[:, 6].max()) * us)
    out = [f"{len(runs)} back-to-back launches, {WG} workgroups each; wall {wall * 1e6:.2f} us per okf_ffn call "
           f"in this run (trace build).  Times in us, medians over the launches.\n",
           "| phase | what ends it | min WG | median WG | max WG |", "|---|---|---:|---:|---:|",
           f"| start spread | last workgroup's start after the first's | | | {np.median(starts):.2f} |"]
    for name, a, b, what in PHASES:
        m = np.median(np.array(rows[name]), axis=0)
        out.append(f"| {name} | {what} | {m[0]:.2f} | {m[1]:.2f} | {m[2]:.2f} |")
    out.append(f"| launch span | first start -> last end | | {np.median(spans):.2f} | |")
    if gaps:
        out.append(f"| gap | last end -> next launch's first start | {np.min(gaps):.2f} | {np.median(gaps):.2f} | "
                   f"{np.max(gaps):.2f} |")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--launches", type=int, default=L)
    ap.add_argument("--lib", help="a library built with OKF_TRACE (default: libokf_quant_trace.so)")
    ap.add_argument("--mfma-only", action="store_true", help="trace ffn_mfma_kernel only")
    args = ap.parse_args()
    n = min(args.launches, L)
    H, D = 6144, 2048

    def rotated(w_np):
        base = torch.from_numpy(w_np).cuda()
        return [base] + [base.clone() for _ in range(max(1, (1 << 30) // w_np.nbytes))]

    gates = rotated(synth.q2_0(H, D, 1002))
    ups = rotated(synth.q2_0(H, D, 1202))
    downs = rotated(synth.q2_0(D, H, 1102))
    gw = [ok.QuantTensor(g, D, H, ok.Q2_0).c() for g in gates]
    uw = [ok.QuantTensor(u, D, H, ok.Q2_0).c() for u in ups]
    dw = [ok.QuantTensor(d, H, D, ok.Q2_0).c() for d in downs]
    refs = [(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d)) for g, u, d in zip(gw, uw, dw)]
    x = torch.from_numpy(synth.activations(1, D, 2002)).cuda()
    h, h2, y = torch.empty(H, device="cuda"), torch.empty(H, device="cuda"), torch.empty(D, device="cuda")
    ptrs = [t.data_ptr() for t in (x, h, h2, y)]
    print("# q2_0_ffn_step_okf_ffn: phase timestamps of the one-launch FFN\n")
    print("Command (run from the repository root on one MI355X, after `python -m chatokf_amd.build --trace`):\n")
    print(f"    python chatokf_amd/trace_ffn.py --launches {n}\n")
    # the context reads OKF_FFN_MFMA when it is created
    variants = (("ffn_mfma_kernel (the default at this shape)", "1"),
                ("ffn_fused_kernel (OKF_FFN_MFMA=0, the VALU digit-plane form)", "0"))
    for title, mf in variants[:1] if args.mfma_only else variants:
        os.environ["OKF_FFN_MFMA"] = mf
        os.environ["OKF_FFN_FUSED"] = "2"  # the one launch, also where two are okf_ffn's default
        enc = ok.Enc(0)
        print(f"## {title}\n")
        print("\n".join(trace(enc, refs, ptrs, n)) + "\n")
        enc.close()


if __name__ == "__main__":
    main()
