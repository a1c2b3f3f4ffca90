#!/usr/bin/env python3
"""Benchmark of the MI355X quantized weight x activation path.

Prints ONE JSON line (the driver contract).  The headline workload is
BASELINE.json configs[1], the Bonsai-1.7B ternary FFN decode step: gate and up
matvecs (Q2_0, W 6144 x 2048) and the down matvec (Q2_0, W 2048 x 6144), one
token.  ``value`` is weight GB/s over that step.  The line also carries the
whole BASELINE suite under ``suite`` (every decode matvec config, the IQ2_XXS
MTP-verify matmul at M = 1 and 4, and the Q4_K pp512 GEMM), each with us per
call, absolute GB/s or TFLOP/s and the roofline fraction.

Timing: inputs are resident in HBM before the timed region.  Every call reads
a different copy of the weights (copies rotated so that >= 1 GiB is cycled,
four times the 256 MB MALL), so weights stream from HBM, not from cache.
Per-call durations come from two HIP events recorded on the library's own
stream around a batch of back-to-back calls (the batch time divided by the
calls, so launch gaps are included and per-event overhead is not); the step
time is bracketed by device synchronisation.

``roofline.traffic`` is read from ``profiles/traffic.json`` when that file holds
a rocprofv3 FETCH_SIZE / WRITE_SIZE measurement of the dominant kernel (made by
running this script under ``rocprofv3 --pmc`` with ``--calibrate``, which adds
plain device copies of known size to scale the counters); otherwise null.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12        # MI355X HBM3E, bytes/s
FP16_PEAK = 2.5e15       # MI355X dense fp16 MFMA, flop/s
ROTATE_BYTES = 1 << 30   # weights cycled per config

METRIC = "quant matvec HBM GB/s (% of 8 TB/s); pp512 Q4_K GEMM TFLOPS (% MFMA)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--suite", default="all", help="'all', 'none' or comma list of suite names")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-headline", action="store_true", help="skip the FFN step (profiling runs)")
    ap.add_argument("--calibrate", action="store_true",
                    help="run 64 MiB device copies first (scale for rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the path has no multi-GPU "
              "mode); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import chatokf_amd as ok
    from chatokf_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()
    enc = ok.Enc(0)
    stream = torch.cuda.ExternalStream(enc.stream)

    def rotated(w_np):
        """Device copies of one weight tensor, enough to cycle >= 1 GiB."""
        base = torch.from_numpy(w_np).cuda()
        n = max(2, -(-ROTATE_BYTES // w_np.nbytes))
        copies = [base] + [base.clone() for _ in range(n - 1)]
        torch.cuda.synchronize()
        return copies

    def time_calls(launch, n_calls, warm, reps=5):
        """Seconds per call: HIP events on enc's stream around `reps` batches of
        n_calls back-to-back launches; returns (mean, best) over the batches."""
        for i in range(warm):
            launch(i)
        per = []
        k = warm
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            # hold the stream for a few ms so the whole batch is queued before
            # the first timed kernel starts: the events then see GPU time only
            with torch.cuda.stream(stream):
                torch.cuda._sleep(20_000_000)
            e0.record(stream)
            for _ in range(n_calls):
                launch(k)
                k += 1
            e1.record(stream)
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) * 1e-3 / n_calls)
        return float(np.mean(per)), float(np.min(per))

    def load_traffic(name):
        path = os.path.join(ROOT, "profiles", "traffic.json")
        if not os.path.exists(path):
            return None
        with open(path) as f:
            t = json.load(f).get(name)
        return None if t is None else int(t["fetch_bytes"] + t["write_bytes"])

    if args.calibrate:
        # a plain elementwise copy of known size (reads 64 MiB, writes 64 MiB)
        # under a kernel name nothing else in this run uses
        src = torch.ones(16 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    rd_buf = torch.empty(ROTATE_BYTES + (64 << 20), dtype=torch.uint8, device="cuda")
    rd_out = torch.zeros(1, dtype=torch.int32, device="cuda")

    def hbm_read_time(nbytes):
        """Seconds per okf_stream_read of nbytes, rotated over rd_buf."""
        nb = nbytes // 16 * 16
        nrot = max(2, ROTATE_BYTES // nb)
        step = (ROTATE_BYTES // nrot) // 256 * 256
        base = rd_buf.data_ptr()
        fn, h, op = enc._lib.okf_stream_read, enc.h, rd_out.data_ptr()

        def call(i):
            fn(h, base + (i % nrot) * step, nb, op)
        return time_calls(call, args.steps, 5)[0]

    hip = ctypes.CDLL("libamdhip64.so")
    cp_dst = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")

    def hbm_copy_time(nbytes):
        """Seconds per device-to-device copy of nbytes (read nbytes, write
        nbytes), the source rotated over rd_buf as the read ceiling's is:
        hipMemcpyAsync on the library's stream, a second, independent method
        beside okf_stream_read for the attainable bandwidth."""
        nb = nbytes // 16 * 16
        nrot = max(2, ROTATE_BYTES // nb)
        step = (ROTATE_BYTES // nrot) // 256 * 256
        base, dst = rd_buf.data_ptr(), cp_dst.data_ptr()
        st = ctypes.c_void_p(enc.stream)

        def call(i):
            hip.hipMemcpyAsync(ctypes.c_void_p(dst), ctypes.c_void_p(base + (i % nrot) * step),
                               ctypes.c_size_t(nb), 3, st)  # hipMemcpyDeviceToDevice
        return time_calls(call, max(20, args.steps // 4), 5)[0]

    cpu_cores = None

    def cpu_config(name, t, M, K, N, ws_np, Xn, xs):
        """The reference's CPU path (oracle restatement of GQ.matvec / GQ.matmul,
        LLM/Gemma/Gemma4Quant.swift:89-170; Q2_0.matvec, LLM/Base/Quant.swift:28-65)
        on this host's cores for one call of the config: median of >= 5 runs
        (one run for the pp512 GEMM)."""
        import oracle  # the CPU baseline leg only

        nonlocal cpu_cores
        if cpu_cores is None:
            cpu_cores = oracle.usable_cores()
        if "silu" in name:
            U = synth.activations(N, K, xs + 100)[0]
            run = lambda: oracle.matvec(t, ws_np[0], K, M, oracle.silu_mul(Xn[0], U), threads=cpu_cores)
        elif len(ws_np) > 1:
            run = lambda: oracle.silu_mul(*[oracle.matvec(t, w, K, M, Xn[0], threads=cpu_cores) for w in ws_np])
        elif N == 1:
            run = lambda: oracle.matvec(t, ws_np[0], K, M, Xn[0], threads=cpu_cores)
        else:
            run = lambda: oracle.matmul(t, ws_np[0], K, M, Xn, threads=cpu_cores)
        reps = 1 if N >= 512 else 5
        ts = []
        for _ in range(reps):
            s0 = time.perf_counter()
            run()
            ts.append(time.perf_counter() - s0)
        return {"cpu_us": round(float(np.median(ts)) * 1e6, 1), "cpu_runs": reps, "cpu_cores": cpu_cores}

    # ----------------------------------------------------------- headline
    t0 = time.time()
    value, step_s, roofline = None, None, None
    K1, M1 = 2048, 6144
    step_bytes = 0
    if not args.no_headline:
        log("bench: generating ternary FFN weights")
        gate_np = synth.q2_0(M1, K1, 1002)
        up_np = synth.q2_0(M1, K1, 1202)
        down_np = synth.q2_0(K1, M1, 1102)
        gates, ups, downs = rotated(gate_np), rotated(up_np), rotated(down_np)
        x = torch.from_numpy(synth.activations(1, K1, 2002)).cuda()
        h = torch.empty(M1, device="cuda")
        h2 = torch.empty(M1, device="cuda")
        y = torch.empty(K1, device="cuda")
        nrot = len(gates)
        step_bytes = gate_np.nbytes + up_np.nbytes + down_np.nbytes

        # the C-ABI calls a host engine makes: weight descriptors built once
        gemv_c = enc.raw_gemv
        gw = [ok.QuantTensor(g, K1, M1, ok.Q2_0).c() for g in gates]
        uw = [ok.QuantTensor(u, K1, M1, ok.Q2_0).c() for u in ups]
        dw = [ok.QuantTensor(d, M1, K1, ok.Q2_0).c() for d in downs]
        xp, hp, h2p, yp = (t.data_ptr() for t in (x, h, h2, y))

        # gate and up in one parallel group, as the reference's FFN encodes
        # them (LLM/Qwen/QwenMetalEngine.swift:918-923, MetalEnc.parallel),
        # then down on silu(gate) * up (siluMul + gemv, :924-928): one
        # okf_ffn call per step (at this shape two launches on the integer
        # matrix cores, gate and up with the SiLU, then down;
        # OKF_FFN_FUSED=2 gives the one launch with a grid barrier)
        pbegin, pend, hctx = enc._lib.okf_parallel_begin, enc._lib.okf_parallel_end, enc.h
        ffn_c = enc._lib.okf_ffn
        refs = [(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d)) for g, u, d in zip(gw, uw, dw)]

        def ffn_step(i):
            gr, ur, dr = refs[i % nrot]
            if ffn_c(hctx, gr, ur, dr, xp, hp, h2p, yp):
                raise RuntimeError("okf_ffn failed")

        for i in range(args.warmup):
            ffn_step(i)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        for i in range(args.steps):
            ffn_step(args.warmup + i)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - w0) / args.steps
        value = step_bytes / step_s / 1e9

        # the two-launch form's kernels, each timed alone: gate and up with the SiLU
        # (okf_gemv_gate_up, one grid), then down on g (okf_gemv)
        gu_c = enc._lib.okf_gemv_gate_up

        def gate_up(i):
            gr, ur, _ = refs[i % nrot]
            gu_c(hctx, gr, ur, xp, hp, h2p)

        step_gpu_t, _ = time_calls(ffn_step, args.steps, 5)
        gate_t, _ = time_calls(gate_up, args.steps, 5)
        down_t, _ = time_calls(lambda i: gemv_c(dw[i % nrot], hp, yp), args.steps, 5)
        fused, q2m = os.environ.get("OKF_FFN_FUSED", "1"), os.environ.get("OKF_Q2_MFMA", "1") != "0"
        if fused == "2" or (fused == "1" and not q2m):
            # okf_ffn is one launch: the step's bytes are the three weight
            # matrices, x, g and u written, g read back, y (ffn_mfma_kernel,
            # or with OKF_FFN_MFMA=0 ffn_fused_kernel)
            ffn_alg = step_bytes + 4 * (K1 + 2 * M1 + M1 + K1)
            kern = "okf::ffn_fused_kernel<Q2_0>" if os.environ.get("OKF_FFN_MFMA", "1") == "0" else \
                "okf::ffn_mfma_kernel<2, 6>"
            dom = ("q2_0_ffn_step_okf_ffn", ffn_alg, step_gpu_t, kern)
        elif gate_t >= down_t:
            dom = ("q2_0_matvec_gate_up_2x6144x2048", gate_np.nbytes + up_np.nbytes, gate_t,
                   "okf::q2m_gemv_kernel<2, 3, true, false, 8, false>" if q2m else "okf::gemv_kernel<Q2_0>")
        else:
            dom = ("q2_0_matvec_2048x6144", down_np.nbytes, down_t,
                   ("okf::q2m_gemv_kernel<4, 1, false, false, 12, true>" if os.environ.get("OKF_Q2_KS", "1") != "0"
                    else "okf::q2m_gemv_kernel<6, 1, false, false, 8, false>") if q2m else "okf::gemv_kernel<Q2_0>")
        roofline = {"kernel": f"{dom[3]} ({dom[0]})", "bound": "hbm",
                    "achieved": round(dom[1] / dom[2] / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(dom[1] / dom[2] / HBM_PEAK, 4),
                    "traffic": load_traffic(dom[0]), "us_per_launch": round(dom[2] * 1e6, 3),
                    "algorithmic_bytes_per_launch": dom[1]}
        log(f"bench: ffn step {step_s*1e6:.2f} us wall ({step_gpu_t*1e6:.2f} us queued), {value:.1f} GB/s; "
            f"gate+up {gate_t*1e6:.2f} us, "
            f"down {down_t*1e6:.2f} us")
        del gates, ups, downs
        torch.cuda.empty_cache()

    # ----------------------------------------------------------- suite
    SUITE = [
        # name, type, M, K, N, weight seed, x seed
        ("q8_0_matvec_2048x2048", ok.Q8_0, 2048, 2048, 1, 1001, 2001),
        ("q2_0_matvec_6144x2048", ok.Q2_0, 6144, 2048, 1, 1002, 2002),
        ("q2_0_matvec_2048x6144", ok.Q2_0, 2048, 6144, 1, 1102, 2102),
        # down on silu(gate) * up (okf_gemv_silu)
        ("q2_0_matvec_silu_2048x6144", ok.Q2_0, 2048, 6144, 1, 1102, 2102),
        # gate and up in one grid with the SiLU (two weight seeds, one x)
        ("q2_0_matvec_gate_up_2x6144x2048", ok.Q2_0, 6144, 2048, 1, (1002, 1202), 2002),
        ("q4_k_matvec_17408x5120", ok.Q4_K, 17408, 5120, 1, 1003, 2003),
        ("q4_k_matmul_17408x5120_m4", ok.Q4_K, 17408, 5120, 4, 1003, 2006),
        ("q4_k_matvec_5120x17408", ok.Q4_K, 5120, 17408, 1, 1103, 2103),
        ("iq2_xxs_matvec_17408x5120_m1", ok.IQ2_XXS, 17408, 5120, 1, 1004, 2004),
        ("iq2_xxs_matmul_17408x5120_m4", ok.IQ2_XXS, 17408, 5120, 4, 1004, 2004),
        ("q4_k_gemm_pp512_17408x5120", ok.Q4_K, 17408, 5120, 512, 1003, 2005),
    ]
    want = None if args.suite == "all" else set(args.suite.split(",")) if args.suite != "none" else set()
    suite = []
    wcache = {}
    for name, t, M, K, N, ws, xs in SUITE:
        if want is not None and name not in want:
            continue
        seeds = ws if isinstance(ws, tuple) else (ws,)
        key = (t, M, K, seeds)
        if key not in wcache:
            wcache.clear()
            torch.cuda.empty_cache()
            log(f"bench: generating {name}")
            ws_np = [synth.weights(t, M, K, sd) for sd in seeds]
            wcache[key] = (sum(w.nbytes for w in ws_np), [rotated(w) for w in ws_np], ws_np)
        wbytes, copies_l, ws_np = wcache[key]
        X = torch.from_numpy(synth.activations(N, K, xs)).cuda()
        Ys = [torch.empty((N, M), device="cuda") for _ in seeds]
        nr = len(copies_l[0])
        wcs_l = [[ok.QuantTensor(c, K, M, t).c() for c in copies] for copies in copies_l]
        xp_, yps = X.data_ptr(), [Y.data_ptr() for Y in Ys]

        if "silu" in name:
            U = torch.from_numpy(synth.activations(N, K, xs + 100)).cuda()

            def call(i, wcs=wcs_l[0], xp_=xp_, up_=U.data_ptr(), yp_=yps[0], nr=nr):
                enc.raw_gemv_silu(wcs[i % nr], xp_, up_, yp_)
        elif len(seeds) == 1:
            def call(i, wcs=wcs_l[0], N=N, xp_=xp_, yp_=yps[0], nr=nr):
                enc.raw_gemm(wcs[i % nr], xp_, N, yp_)
        else:  # gate and up in one grid with the SiLU (okf_gemv_gate_up)
            grefs = [(ctypes.byref(a), ctypes.byref(b)) for a, b in zip(*wcs_l)]

            def call(i, grefs=grefs, xp_=xp_, yps=yps, nr=nr):
                gr, ur = grefs[i % nr]
                if enc._lib.okf_gemv_gate_up(enc.h, gr, ur, xp_, yps[0], yps[1]):
                    raise RuntimeError("okf_gemv_gate_up failed")

        n_calls = args.steps if N < 512 else max(10, args.steps // 10)
        mean_s, med_s = time_calls(call, n_calls, max(3, args.warmup // 2))  # (mean, best batch)
        flops = 2.0 * M * K * N
        rec = {"name": name, "us": round(mean_s * 1e6, 3), "us_best": round(med_s * 1e6, 3),
               "weight_bytes": wbytes, "GBps": round(wbytes / mean_s / 1e9, 1),
               "TFLOPs": round(flops / mean_s / 1e12, 2)}
        if N >= 512:
            rec["bound"], rec["frac"] = "mfma_fp16", round(flops / mean_s / FP16_PEAK, 4)
        else:
            rec["bound"], rec["frac"] = "hbm", round(wbytes / mean_s / HBM_PEAK, 4)
            # the attainable single-launch ceiling: a plain streaming read of
            # the same number of bytes, rotated over the same >= 1 GiB
            rd_s = hbm_read_time(wbytes)
            rec["hbm_read_us"] = round(rd_s * 1e6, 3)
            rec["hbm_read_frac"] = round(wbytes / rd_s / HBM_PEAK, 4)
            if wbytes <= cp_dst.numel():
                # the same bytes copied by hipMemcpyAsync: (read + write) / time
                cp_s = hbm_copy_time(wbytes)
                rec["hbm_copy_us"] = round(cp_s * 1e6, 3)
                rec["hbm_copy_frac"] = round(2 * wbytes / cp_s / HBM_PEAK, 4)
            # warm: the same call on one weight copy (L2 / MALL resident after the
            # first call; reported beside, not the measurement)
            warm_s, _ = time_calls(lambda i: call(0), n_calls, 3)
            rec["us_warm"] = round(warm_s * 1e6, 3)
        if not args.no_cpu:
            rec.update(cpu_config(name, t, M, K, N, ws_np, X.cpu().numpy(), xs))
        log("bench:", json.dumps(rec))
        suite.append(rec)
        del X, Ys
    wcache.clear()

    # the attainable bandwidth, two independent methods at two sizes: the
    # library's plain streaming read and hipMemcpyAsync (a copy moves 2x its
    # size), rotated over the same >= 1 GiB
    if want is None or "hbm_ceiling" in want:
        rec = {"name": "hbm_ceiling", "bound": "hbm"}
        for mb in (50, 512):
            nb = mb * 1000 * 1000
            if nb > cp_dst.numel():
                cp_dst = torch.empty(nb, dtype=torch.uint8, device="cuda")
            rd_s, cp_s = hbm_read_time(nb), hbm_copy_time(nb)
            rec[f"read_{mb}MB_us"] = round(rd_s * 1e6, 3)
            rec[f"read_{mb}MB_frac"] = round(nb / rd_s / HBM_PEAK, 4)
            rec[f"copy_{mb}MB_us"] = round(cp_s * 1e6, 3)
            rec[f"copy_{mb}MB_frac"] = round(2 * nb / cp_s / HBM_PEAK, 4)
        log("bench:", json.dumps(rec))
        suite.append(rec)

    # the FFN's neighbours: add + RMSNorm over a pp512 batch (x, r, w read,
    # x and y written) and argmax over one 248320-wide vocabulary row
    NEIGH = [("add_rmsnorm_512x5120", 512, 5120), ("argmax_rows_1x248320", 1, 248320)]
    for name, rows, n in NEIGH:
        if want is not None and name not in want:
            continue
        g = torch.Generator(device="cuda").manual_seed(7)
        xs_ = [torch.randn(rows, n, device="cuda", generator=g) for _ in range(max(2, ROTATE_BYTES // (rows * n * 4)))]
        nr = len(xs_)
        if name.startswith("add"):
            r_ = torch.randn(rows, n, device="cuda", generator=g)
            w_ = torch.rand(n, device="cuda", generator=g) + 0.5
            y_ = torch.empty(rows, n, device="cuda")
            fn, args_ = enc._lib.okf_add_rmsnorm_batch, (r_.data_ptr(), w_.data_ptr(), y_.data_ptr())
            nbytes = (4 * rows + 1) * n * 4  # x, r read; x, y written; w read once

            def call(i, xs_=xs_, nr=nr):
                if fn(enc.h, xs_[i % nr].data_ptr(), *args_, n, rows, ctypes.c_float(1e-6)):
                    raise RuntimeError("okf_add_rmsnorm_batch failed")
        else:
            o_ = torch.empty(rows, dtype=torch.int32, device="cuda")
            nbytes = rows * n * 4

            def call(i, xs_=xs_, nr=nr):
                if enc._lib.okf_argmax_rows(enc.h, xs_[i % nr].data_ptr(), n, rows, o_.data_ptr()):
                    raise RuntimeError("okf_argmax_rows failed")
        mean_s, best_s = time_calls(call, args.steps, max(3, args.warmup // 2))
        rec = {"name": name, "us": round(mean_s * 1e6, 3), "us_best": round(best_s * 1e6, 3),
               "bytes": nbytes, "GBps": round(nbytes / mean_s / 1e9, 1), "bound": "hbm",
               "frac": round(nbytes / mean_s / HBM_PEAK, 4)}
        log("bench:", json.dumps(rec))
        suite.append(rec)
        del xs_

    # ----------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu and not args.no_headline:
        import oracle  # the CPU baseline leg: the oracle restatement of GQ.matvec

        cores = oracle.usable_cores()
        xn = synth.activations(1, K1, 2002)[0]
        times = []
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds or len(times) < 5:
            s = time.perf_counter()
            gn = oracle.matvec(ok.Q2_0, gate_np, K1, M1, xn, threads=cores)
            un = oracle.matvec(ok.Q2_0, up_np, K1, M1, xn, threads=cores)
            oracle.matvec(ok.Q2_0, down_np, M1, K1, oracle.silu_mul(gn, un), threads=cores)
            times.append(time.perf_counter() - s)
        cpu_step = float(np.median(times))
        cpu = {"value": round(step_bytes / cpu_step / 1e9, 2), "unit": "GB/s", "cores": cores,
               "kind": "port",
               "sample": f"median of {len(times)} ternary FFN steps (gate, up, silu*mul, down; "
                         f"same inputs) in {time.perf_counter() - c0:.1f} s: C restatement of "
                         "Q2_0.matvec (LLM/Base/Quant.swift:28-65), row-parallel over cores",
               "us_per_step": round(cpu_step * 1e6, 1)}
        log("bench: cpu", json.dumps(cpu))

    out = {
        "metric": METRIC,
        "value": None if value is None else round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None if step_s is None else round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 activations (exact 23-bit integers per 32-weight group) x integer weight codes "
                 "(int8 dot4, exact per group), f32 scales and accumulation",
        "data": "synthetic (reference LCG, BASELINE.json distributions); weights rotated over >= 1 GiB",
        "config": {"workload": "BASELINE configs[1]: Bonsai-1.7B ternary FFN decode step, one token "
                               "(one okf_ffn call): gate+up Q2_0 W 6144x2048 with the siluMul "
                               "(as the reference's parallel group + in-place siluMul), then down "
                               "Q2_0 W 2048x6144 on silu(gate)*up: two launches on the integer "
                               "matrix cores",
                   "weight_bytes_per_step": step_bytes, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "suite": suite,
        "wall_s": round(time.time() - t0, 1),
    }
    enc.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
