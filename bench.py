#!/usr/bin/env python3
"""Benchmark of the MI355X scaled-GEMM hot path (one GPU).

Headline (``value``): MXFP4 x MXFP4 (A4W4) GEMM at M=N=K=8192 (BASELINE.json
configs[2]) in TFLOP/s: A, B drawn N(0,1) from a seed, quantised per 1x32 to
MXFP4 (e2m1 + e8m0, Even rounding as the reference test/tuner), B
preshuffled, bf16 output.  One step = one ``gemm_a4w4_asm`` call (the entry
``gemm_a4w4`` dispatches to) on inputs resident in HBM, into a preallocated
output.  The K timed steps are captured in a HIP graph and replayed once
between two synchronisations (launch overhead is not part of a step), after
W warm-up steps replayed through the same graph for at least one second
(the clocks ramp up under load).

Also reported on the same JSON line:
* ``decode``: the bandwidth-bound configs[1] (M in {1,8,16,32,64}, N=7168,
  K=2048), cold-cache (B/scales rotated over >512 MiB) and warm, GB/s incl.
  scales and % of 8 TB/s;
* ``decode_sweep`` / ``prefill_sweep``: the dispatch sweep, M in
  {1, 32} cold and M in {256, 2048, 8192} warm, A4W4 (also with the
  activation quantised on the fly) and bf16, through the tuned dispatch;
* ``a8w4_mxfp8``: configs[3], MXFP8 x MXFP4 at M in {256, 4096}, N=7168,
  K=16384, the GEMM alone and with the dynamic MXFP8 quant of a bf16 input;
* ``extra``: bf16 A16W16 8192x8192x8192 (row-major and preshuffled B), the
  K=16384 prefill variant, the quantisers and the "next" rows;
* ``roofline`` of the dominant kernel (A4W4 tile kernel) from HIP events on the
  launch stream; ``traffic`` is the HBM bytes/launch measured with rocprofv3
  PMC counters (profiles/), or null when no such measurement is committed;
* ``cpu_baseline``: the reference's CPU torch path on the full headline
  problem (dequantise to f32 + ``torch.mm``, op_tests/test_gemm_a4w4.py:23-39,
  restated in oracle/torch_ref.py), dequantisation and matmul timed apart.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MXFP4 = 10100.0   # TFLOP/s dense (MI355X)
PEAK_MXFP8 = 5000.0
PEAK_BF16 = 2500.0
PEAK_HBM = 8000.0      # GB/s
COPY_BYTES = 1 << 30    # calibration copy of the traffic counter runs
REF_A4W4_8192 = 5089.97  # TFLOP/s, aiter/configs/a4w4_blockscale_tuned_gemm.csv:1284


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def quantised_operands(m, n, k, seed, dev):
    import aiter_amd

    g = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn((m, k), generator=g, dtype=torch.float32).to(dev)
    b = torch.randn((n, k), generator=g, dtype=torch.float32).to(dev)
    aq, as_ = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
    bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
    del a, b
    return aq, as_, aiter_amd.shuffle_weight(bq), bs


def time_graph(fn, steps, warmup, min_warm_s=0.3):
    """Capture `steps` calls of fn() in a HIP graph and time one replay with
    HIP events on the launch stream; returns seconds per call.

    Warm-up: `warmup` calls, replayed through the same graph (whole replays,
    at least one), continued until `min_warm_s` of GPU work has run.  MI355X
    raises its clocks over the first few hundred milliseconds of load, so a
    cold measurement reads up to 20% slow."""
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # one eager call on the capture stream (lazy state, workspaces)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(steps):
                fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    done = 0
    while done < max(warmup, 1) or time.perf_counter() - t0 < min_warm_s:
        g.replay()
        done += steps
        torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        e0.record(s)
        g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / steps


def a4w4_bytes(m, n, k):
    """Algorithmic HBM bytes incl. scales: A, B (1/2 B/elem), both e8m0 scale
    tensors (1 B per 32 elems), bf16 C."""
    return m * k // 2 + n * k // 2 + m * k // 32 + n * k // 32 + 2 * m * n


def headline_kernel():
    """The instance gemm_a4w4 dispatches M=N=K=8192 to: the tuned table's
    kernelName, else "" (the library heuristic)."""
    import aiter_amd

    cfg = aiter_amd.get_GEMM_config(8192, 8192, 8192)
    return str(cfg["kernelName"]) if cfg else ""


def bench_prefill(steps, warmup, dev):
    import aiter_amd

    m = n = k = 8192
    aq, as_, bq, bs = quantised_operands(m, n, k, 0, dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    kname = headline_kernel()

    def step():
        aiter_amd.gemm_a4w4_asm(aq, bq, as_, bs, out, kernelName=kname)

    sec = time_graph(step, steps, warmup, min_warm_s=1.0)
    flop = 2.0 * m * n * k
    return sec, flop / sec / 1e12, kname


_CEIL = {}


# launch shapes of the calibration read (grid, threads per workgroup, loads
# in flight per thread): the fastest ones of a sweep over unroll 1-8, block
# 256-1024, grid 256-4096 and the cache policies, at 7.8, 29 and 125 MB
CEILING_SHAPES = ((2048, 256, 1), (4096, 512, 1), (512, 1024, 1), (1024, 256, 4))


def read_ceiling(dev, nbytes):
    """Seconds per call of the fastest calibration streaming read
    (`hbm_stream_read_cfg`, nothing but 16-byte loads) over ``nbytes``, cold:
    the buffers rotate through > 512 MiB.  The attainable HBM read time at
    that byte count, launch and ramp included, that a bandwidth-bound GEMM is
    compared to (the minimum over CEILING_SHAPES)."""
    from aiter_amd._lib import call

    n = (nbytes + 15) // 16 * 16
    if n not in _CEIL:
        copies = max(2, -(-(600 << 20) // n))
        bufs = [torch.ones(n, dtype=torch.uint8, device=dev) for _ in range(copies)]
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        best = None
        for grid, block, unroll in CEILING_SHAPES:
            it = {"i": 0}

            def run():
                b = bufs[it["i"] % copies]
                it["i"] += 1
                call("hbm_stream_read_cfg", b, sink, grid, block, unroll, -1)

            t = time_graph(run, copies * (4 if copies <= 100 else 1), 3)
            best = t if best is None else min(best, t)
        _CEIL[n] = best
        del bufs
    return _CEIL[n]


def launch_floor(dev):
    """Seconds per graph-replayed launch of an empty grid of 1024 workgroups
    (hbm_stream_read_cfg policy -2): the floor under any single-launch call."""
    from aiter_amd._lib import call

    src = torch.ones(1 << 20, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    return time_graph(lambda: call("hbm_stream_read_cfg", src, sink, 1024, 256, 1, -2), 100, 3)


def bench_decode(dev, steps=50):
    import aiter_amd

    res = []
    n, k = 7168, 2048
    g = torch.Generator(device="cpu").manual_seed(1)
    b = torch.randn((n, k), generator=g).to(dev)
    bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
    bq = aiter_amd.shuffle_weight(bq)
    per = bq.numel() + bs.numel()
    copies = max(2, (600 << 20) // per)  # rotate > 512 MiB (defeats L2 + 256 MiB MALL)
    bqs = [bq.clone() for _ in range(copies)]
    bss = [bs.clone() for _ in range(copies)]
    for m in (1, 8, 16, 32, 64):
        a = torch.randn((m, k), generator=g).to(dev)
        aq, as_ = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
        out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=dev)
        it = {"i": 0}

        # the kernel gemm_a4w4 dispatches to (tuned table, else the heuristic),
        # called on a preallocated output
        cfg = aiter_amd.get_GEMM_config(m, n, k)
        kname = str(cfg["kernelName"]) if cfg else ""
        l2 = int(cfg.get("splitK", 0) or 0) if cfg else 0

        def cold():
            i = it["i"] % copies
            it["i"] += 1
            aiter_amd.gemm_a4w4_asm(aq, bqs[i], as_, bss[i], out, kernelName=kname, log2_k_split=l2)

        def warm():
            aiter_amd.gemm_a4w4_asm(aq, bq, as_, bs, out, kernelName=kname, log2_k_split=l2)

        t_cold = time_graph(cold, min(steps, copies), 3)
        t_warm = time_graph(warm, steps, 3)
        byts = a4w4_bytes(m, n, k)
        t_ceil = read_ceiling(dev, byts)
        t_floor = launch_floor(dev) if not res else res[0]["launch_floor_us"] * 1e-6
        ref_bw = (m * k / 2 + n * k / 2 + 2 * m * n)  # reference `bw` formula (scales excluded)
        res.append({
            "M": m, "N": n, "K": k, "kernel": kname or "heuristic",
            "us_cold": round(t_cold * 1e6, 3), "us_warm": round(t_warm * 1e6, 3),
            "GBps_cold": round(byts / t_cold / 1e9, 1), "GBps_warm": round(byts / t_warm / 1e9, 1),
            "hbm_frac_cold": round(byts / t_cold / 1e9 / PEAK_HBM, 4),
            "ref_formula_GBps_cold": round(ref_bw / t_cold / 1e9, 1),
            "read_ceiling_us": round(t_ceil * 1e6, 3), "frac_of_read_ceiling": round(t_ceil / t_cold, 4),
            "launch_floor_us": round(t_floor * 1e6, 3),
        })
        log(f"decode M={m}: cold {t_cold*1e6:.2f} us ({byts/t_cold/1e9:.0f} GB/s), warm {t_warm*1e6:.2f} us")
    return res


SWEEP_NK = ((4096, 4096), (14336, 4096), (4096, 14336), (28672, 8192), (8192, 28672))


def bench_decode_sweep(dev, ms=(1, 32)):
    """Decode rows of the dispatch sweep: M in {1, 32}
    over its five (N, K), A4W4 (MXFP4 activations, preshuffled B) and bf16,
    cold: the weights rotate through > 512 MiB of copies so every call reads
    them from HBM.  GB/s counts A, B, their scales and C once;
    ``frac_of_read_ceiling`` = the calibration read's time over as many bytes
    / the GEMM's time."""
    import aiter_amd

    rows = []
    g = torch.Generator(device="cpu").manual_seed(3)
    for n, k in SWEEP_NK:
        b = torch.randn((n, k), generator=g).to(dev)
        bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
        bq = aiter_amd.shuffle_weight(bq)
        b16 = b.to(torch.bfloat16)
        del b
        for fam in ("a4w4", "bf16"):
            per = bq.numel() + bs.numel() if fam == "a4w4" else b16.numel() * 2
            copies = max(2, -(-(600 << 20) // per))
            if fam == "a4w4":
                ws = [(bq.clone(), bs.clone()) for _ in range(copies)]
            else:
                ws = [b16.clone() for _ in range(copies)]
            for m in ms:
                a = torch.randn((m, k), generator=g).to(dev)
                it = {"i": 0}
                if fam == "a4w4":
                    aq, as_ = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
                    cfg = aiter_amd.get_GEMM_config(m, n, k)
                    kname = str(cfg["kernelName"]) if cfg else ""
                    l2 = int(cfg.get("splitK", 0) or 0) if cfg else 0
                    out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=dev)
                    byts = a4w4_bytes(m, n, k)

                    def cold():
                        w, sc = ws[it["i"] % copies]
                        it["i"] += 1
                        aiter_amd.gemm_a4w4_asm(aq, w, as_, sc, out, kernelName=kname, log2_k_split=l2)
                else:
                    a16 = a.to(torch.bfloat16)
                    kname = "tuned/heuristic"
                    byts = 2 * (m * k + n * k + m * n)

                    def cold():
                        w = ws[it["i"] % copies]
                        it["i"] += 1
                        aiter_amd.gemm_a16w16(a16, w)
                t = time_graph(cold, copies * 4, 3)
                t_ceil = read_ceiling(dev, byts)
                rows.append({"fam": fam, "M": m, "N": n, "K": k, "kernel": kname or "heuristic",
                             "us_cold": round(t * 1e6, 2), "GBps_cold": round(byts / t / 1e9, 1),
                             "hbm_frac_cold": round(byts / t / 1e9 / PEAK_HBM, 4),
                             "read_ceiling_us": round(t_ceil * 1e6, 2),
                             "frac_of_read_ceiling": round(t_ceil / t, 4)})
                log(f"decode sweep {fam} M={m} N={n} K={k}: {t*1e6:.2f} us, {byts/t/1e9:.0f} GB/s")
            del ws
        del bq, bs, b16
        torch.cuda.empty_cache()
    return rows


def bench_prefill_sweep(dev, ms=(256, 2048, 8192)):
    """Compute-bound rows of the dispatch sweep: M in
    {256, 2048, 8192} over its five (N, K), through the tuned dispatch.
    A4W4: ``gemm_a4w4`` on MXFP4 operands (``us``), and with the bf16
    activation quantised on the fly first (``us_with_quant``:
    dynamic_mxfp4_quant + gemm_a4w4); bf16: ``gemm_a16w16`` with row-major B
    (the layout of the reference's bf16 rows).  Warm L2; roofline fraction
    against the dense MXFP4 / bf16 peak."""
    import aiter_amd

    rows = []
    g = torch.Generator(device=dev).manual_seed(5)
    for n, k in SWEEP_NK:
        w16 = torch.randn((n, k), generator=g, device=dev).to(torch.bfloat16)
        wq, ws = aiter_amd.dynamic_mxfp4_quant(w16, shuffle=True)
        wq = aiter_amd.shuffle_weight(wq)
        for m in ms:
            x16 = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
            xq, xs = aiter_amd.dynamic_mxfp4_quant(x16, shuffle=True)
            flop = 2.0 * m * n * k
            steps = max(3, min(20, int(2e13 / flop)))
            cfg = aiter_amd.get_GEMM_config(m, n, k)
            t = time_graph(lambda: aiter_amd.gemm_a4w4(xq, wq, xs, ws), steps, 2)
            tq = time_graph(lambda: _quant_then_gemm(aiter_amd, x16, wq, ws), steps, 2)
            rows.append({"fam": "a4w4", "M": m, "N": n, "K": k,
                         "kernel": str(cfg["kernelName"]) if cfg else "heuristic",
                         "us": round(t * 1e6, 2), "TFLOPs": round(flop / t / 1e12, 1),
                         "frac_mxfp4_peak": round(flop / t / 1e12 / PEAK_MXFP4, 4),
                         "us_with_quant": round(tq * 1e6, 2)})
            log(f"prefill sweep a4w4 M={m} N={n} K={k}: {t*1e6:.1f} us ({flop/t/1e12:.0f} TF), "
                f"with quant {tq*1e6:.1f} us")
            t16 = time_graph(lambda: aiter_amd.gemm_a16w16(x16, w16), steps, 2)
            rows.append({"fam": "bf16", "M": m, "N": n, "K": k, "kernel": "tuned/heuristic",
                         "us": round(t16 * 1e6, 2), "TFLOPs": round(flop / t16 / 1e12, 1),
                         "frac_bf16_peak": round(flop / t16 / 1e12 / PEAK_BF16, 4)})
            log(f"prefill sweep bf16 M={m} N={n} K={k}: {t16*1e6:.1f} us ({flop/t16/1e12:.0f} TF)")
            del x16, xq, xs
        del w16, wq, ws
        torch.cuda.empty_cache()
    return rows


def _quant_then_gemm(aiter_amd, x16, wq, ws):
    xq, xs = aiter_amd.dynamic_mxfp4_quant(x16, shuffle=True)
    return aiter_amd.gemm_a4w4(xq, wq, xs, ws)


def bench_a8w4(dev, ms=(256, 4096)):
    """MXFP8 x MXFP4, M in {256, 4096}, N = 7168,
    K = 16384, from a bf16 N(0,1) activation: the GEMM alone on quantised
    operands and the whole call with the dynamic MXFP8 quant
    (``gemm_a8w4_mxfp8_dynamic``: quant kernel + GEMM), against the dense
    MXFP8 peak."""
    import aiter_amd

    rows = []
    n, k = 7168, 16384
    g = torch.Generator(device=dev).manual_seed(7)
    w = torch.randn((n, k), generator=g, device=dev).to(torch.bfloat16)
    wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
    wq = aiter_amd.shuffle_weight(wq)
    del w
    for m in ms:
        x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
        xq, xs = aiter_amd.dynamic_mxfp8_quant(x, shuffle=True)
        flop = 2.0 * m * n * k
        t = time_graph(lambda: aiter_amd.gemm_a8w4_mxfp8(xq, wq, xs, ws, a_preshuffle=False), 10, 2)
        td = time_graph(lambda: aiter_amd.gemm_a8w4_mxfp8_dynamic(x, wq, ws), 10, 2)
        tq = time_graph(lambda: aiter_amd.dynamic_mxfp8_quant(x, shuffle=True), 20, 2)
        cfg = aiter_amd.gemm_op_a8w4.get_GEMM_A8W4_config(m, n, k)
        rows.append({"M": m, "N": n, "K": k, "kernel": str(cfg["kernelName"]) if cfg else "heuristic",
                     "gemm_us": round(t * 1e6, 1), "gemm_TFLOPs": round(flop / t / 1e12, 1),
                     "frac_mxfp8_peak": round(flop / t / 1e12 / PEAK_MXFP8, 4),
                     "with_dynamic_quant_us": round(td * 1e6, 1),
                     "with_dynamic_quant_TFLOPs": round(flop / td / 1e12, 1),
                     "quant_us": round(tq * 1e6, 1), "quant_GBps": round(m * k * (2 + 1 + 1 / 32) / tq / 1e9, 1)})
        log(f"a8w4 M={m}: gemm {t*1e6:.1f} us ({flop/t/1e12:.0f} TF), with dynamic quant {td*1e6:.1f} us")
        del x, xq, xs
    return rows


def bench_extra(dev):
    import aiter_amd

    out = {}
    # bf16 A16W16 M=N=K=8192 through the tuned dispatch (gemm_a16w16 / tgemm.mm),
    # row-major B and preshuffled B
    m = n = k = 8192
    g = torch.Generator(device="cpu").manual_seed(2)
    a = torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn((n, k), generator=g).to(torch.bfloat16).to(dev)
    bs = aiter_amd.shuffle_weight(b)
    for tag, w in (("bf16_8192x8192x8192", b), ("bf16_8192x8192x8192_bpreshuffle", bs)):
        t = time_graph(lambda w=w: aiter_amd.gemm_a16w16(a, w), 10, 2)
        out[tag] = {"us": round(t * 1e6, 1), "TFLOPs": round(2 * m * n * k / t / 1e12, 1),
                    "frac_bf16_peak": round(2 * m * n * k / t / 1e12 / PEAK_BF16, 4)}
    del a, b, bs
    out["bf16_cpu_plumbing"] = bf16_plumbing(dev)
    # A4W4 prefill, the K=16384, N=2048 variant of BASELINE configs[2]
    m, n, k = 8192, 2048, 16384
    aq, as_, bq, bs_ = quantised_operands(m, n, k, 6, dev)
    t = time_graph(lambda: aiter_amd.gemm_a4w4(aq, bq, as_, bs_), 20, 2)
    cfg = aiter_amd.get_GEMM_config(m, n, k)
    out["a4w4_8192x2048x16384"] = {"us": round(t * 1e6, 1), "TFLOPs": round(2 * m * n * k / t / 1e12, 1),
                                   "frac_mxfp4_peak": round(2 * m * n * k / t / 1e12 / PEAK_MXFP4, 4),
                                   "kernel": str(cfg["kernelName"]) if cfg else "heuristic"}
    del aq, as_, bq, bs_
    # MXFP4 activation quant 8192 x 8192 bf16
    xa = torch.randn((8192, 8192), generator=g).to(torch.bfloat16).to(dev)
    tq = time_graph(lambda: aiter_amd.per_1x32_mx_quant_hip(xa, shuffle=True), 20, 2)
    out["mxfp4_quant_8192x8192"] = {"us": round(tq * 1e6, 1),
                                    "GBps": round(8192 * 8192 * (2 + 0.5 + 1 / 32) / tq / 1e9, 1)}
    # fused RMSNorm -> MXFP4 quant prologue vs RMSNorm (torch, bf16 out) then the quantiser
    wa = torch.randn(8192, generator=g).to(torch.bfloat16).to(dev)
    tf = time_graph(lambda: aiter_amd.fused_rms_mxfp4_quant(xa, wa, 1e-6, shuffle=True), 20, 2)
    tu = time_graph(lambda: aiter_amd.per_1x32_mx_quant_hip(
        torch.nn.functional.rms_norm(xa, (8192,), wa, eps=1e-6), shuffle=True), 20, 2)
    out["fused_rms_mxfp4_quant_8192x8192"] = {"us": round(tf * 1e6, 1),
                                              "GBps": round(8192 * 8192 * (2 + 0.5 + 1 / 32) / tf / 1e9, 1),
                                              "unfused_us": round(tu * 1e6, 1)}
    del xa
    # low-precision outputs of the 8192^3 A4W4 GEMM (e2m1 / MXFP8), against the bf16-output call
    aq, as_, bq, bs_ = quantised_operands(8192, 8192, 8192, 4, dev)
    t16 = time_graph(lambda: aiter_amd.gemm_a4w4(aq, bq, as_, bs_), 10, 2)
    for tag, fn in (("a4w4o4_8192x8192x8192", aiter_amd.gemm_a4w4o4), ("a4w4o8_8192x8192x8192", aiter_amd.gemm_a4w4o8)):
        t = time_graph(lambda fn=fn: fn(aq, bq, as_, bs_), 10, 2)
        out[tag] = {"us": round(t * 1e6, 1), "TFLOPs": round(2 * 8192 ** 3 / t / 1e12, 1),
                    "bf16_out_us": round(t16 * 1e6, 1)}
    del aq, as_, bq, bs_
    # batched bf16 (op_tests/test_batched_gemm_bf16.py defaults: b = 16, N = 1024, K = 4096):
    # one batched launch against a loop of per-batch calls
    bt = []
    for mb in (1, 32, 512):
        xb = torch.randn((16, mb, 4096), generator=g).to(torch.bfloat16).to(dev)
        wb = torch.randn((16, 1024, 4096), generator=g).to(torch.bfloat16).to(dev)
        yb = torch.empty((16, mb, 1024), dtype=torch.bfloat16, device=dev)
        t = time_graph(lambda: aiter_amd.batched_gemm_bf16(xb, wb, yb), 10, 2)
        tl = time_graph(lambda: [aiter_amd.gemm_a16w16(xb[i], wb[i]) for i in range(16)], 10, 2)
        flop = 2 * 16 * mb * 1024 * 4096
        bt.append({"b": 16, "M": mb, "N": 1024, "K": 4096, "us": round(t * 1e6, 1),
                   "TFLOPs": round(flop / t / 1e12, 1), "GBps": round(2 * 16 * (mb * 4096 + 1024 * 4096 + mb * 1024) / t / 1e9, 1),
                   "loop_us": round(tl * 1e6, 1)})
    out["batched_bf16"] = bt
    out["fused_gemm_afp4wfp4_a16w16"] = bench_fused_a16w16(dev)
    out["fused_moe_a4w4_deepseek"] = bench_moe(dev)
    return out


def bench_fused_a16w16(dev, ms=(1, 16, 64), n4=4096, n16=256, k=7168):
    """fused_gemm_afp4wfp4_a16w16 (an MXFP4 gate-up projection and the bf16
    router of one layer over the same activations; DeepSeek-like N = 4096 and
    256 experts, K = 7168): one grid over both GEMMs' column blocks at decode
    sizes, against the two GEMMs called one after the other."""
    import aiter_amd

    g = torch.Generator(device="cpu").manual_seed(12)
    res = []
    for m in ms:
        a = torch.randn((m, k), generator=g).to(dev)
        w = torch.randn((n4, k), generator=g).to(dev)
        wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
        wq = aiter_amd.shuffle_weight(wq)
        aq, as_sh = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
        _, as_pl = aiter_amd.dynamic_mxfp4_quant(a, shuffle=False)
        xb = a.to(torch.bfloat16)
        wb = torch.randn((n16, k), generator=g).to(torch.bfloat16).to(dev)
        # the preshuffled op's layouts: w [N/16, K*8], scales [rows/32, K], x scales plain below 32 rows
        w_t = wq.view(torch.uint8).view(n4 // 16, k * 8)
        ws_t = ws.view(torch.uint8).view(-1, k)
        xs_t = as_sh.view(torch.uint8).view(-1, k) if m >= 32 else as_pl
        fused = lambda: aiter_amd.fused_gemm_afp4wfp4_a16w16(aq, w_t, xs_t, ws_t, xb, wb, is_fp4_preshuffled=True)
        apart = lambda: (aiter_amd.gemm_a4w4(aq, wq, as_sh, ws), aiter_amd.gemm_a16w16(xb, wb))
        t = time_graph(fused, 20, 2)
        t2 = time_graph(apart, 20, 2)
        res.append({"M": m, "N_fp4": n4, "N_bf16": n16, "K": k, "us": round(t * 1e6, 2),
                    "two_calls_us": round(t2 * 1e6, 2)})
        log(f"fused_gemm_afp4wfp4_a16w16 {res[-1]}")
    return res


def bench_moe(dev, tokens=(1, 16, 128, 1024, 4096), model="deepseek"):
    """fused_moe A4W4 at the reference test's DeepSeek shape (op_tests/test_moe_2stage.py
    defaults: model_dim 7168, inter_dim 256, 257 experts, topk 9), graph-captured
    so that host time is excluded.  Weights are random fp4 bytes with scale
    bytes near 2^-6 (preshuffled); routing softmax-top-9 of random scores.
    Roofline: HBM bytes of the experts a call touches (w1 + w2 + scales, each
    read once) and of the activations, against 8 TB/s; FLOPs against the
    dense MXFP4 peak."""
    import aiter_amd

    E, topk, dim, inter = MOE_MODELS[model]
    g = torch.Generator(device=dev).manual_seed(11)
    w1 = torch.randint(0, 256, (E * 2 * inter, dim // 2), dtype=torch.uint8, device=dev, generator=g)
    w2 = torch.randint(0, 256, (E * dim, inter // 2), dtype=torch.uint8, device=dev, generator=g)
    w1s = aiter_amd.shuffle_scale(torch.randint(119, 123, (E * 2 * inter, dim // 32), dtype=torch.uint8, device=dev,
                                                generator=g))
    w2s = aiter_amd.shuffle_scale(torch.randint(119, 123, (E * dim, inter // 32), dtype=torch.uint8, device=dev,
                                                generator=g))
    w1 = aiter_amd.shuffle_weight(w1).view(E, 2 * inter, dim // 2)
    w2 = aiter_amd.shuffle_weight(w2).view(E, dim, inter // 2)
    per_expert = 2 * inter * dim // 2 + dim * inter // 2 + 2 * inter * dim // 32 + dim * inter // 32
    out = []
    for m in tokens:
        x = torch.randn(m, dim, device=dev, generator=g).to(torch.bfloat16)
        tw, ti = torch.topk(torch.softmax(torch.randn(m, E, device=dev, generator=g), -1), topk, -1)
        tw = (tw / tw.sum(-1, keepdim=True)).float()
        ti = ti.to(torch.int32)
        fn = lambda: aiter_amd.fused_moe(x, w1, w2, tw, ti, quant_type=aiter_amd.QuantType.per_1x32, w1_scale=w1s,
                                         w2_scale=w2s)
        t = time_graph(fn, 10, 2)
        stages = _moe_stage_times(aiter_amd, x, w1, w2, w1s, w2s, tw, ti, E, topk, dim, inter, REF_MOE[model])
        touched = int(torch.unique(ti).numel())
        nbytes = touched * per_expert + m * dim * 2 * 2
        flop = 2 * m * topk * (2 * inter * dim + dim * inter)
        out.append({"tokens": m, "us": round(t * 1e6, 1), "TFLOPs": round(flop / t / 1e12, 1),
                    "frac_mxfp4_peak": round(flop / t / 1e12 / PEAK_MXFP4, 4), "experts_touched": touched,
                    "GBps": round(nbytes / t / 1e9, 1), "frac_hbm": round(nbytes / t / 1e9 / PEAK_HBM, 4),
                    "block_m": aiter_amd.get_block_size_M(m, topk, E, inter), **stages})
        log(f"fused_moe {model} tokens={m}: {out[-1]}")
    return out


# the reference's tuned stage times (us1, us2) at model_dim 7168, inter_dim 256,
# 257 experts, topk 9: aiter/configs/model_configs/dsv3_fp4_tuned_fmoe.csv:2,6,9,12,14
REF_MOE_STAGES = {1: (11.3537, 7.5406), 16: (40.5338, 24.9519), 128: (87.5346, 54.4124),
                  1024: (106.2571, 107.529), 4096: (191.9986, 283.9092)}

# (experts, topk, model_dim, inter_dim) of the models whose MXFP4 fused-MoE
# rows the reference tunes, and their tuned (us1, us2) at 1/16/128/1024/4096
# tokens (rows 2, 6, 9, 12, 14 of each file; Qwen3.5's 1- and 16-token rows
# are one-stage kernels: us2 0, us1 the whole call)
MOE_MODELS = {"deepseek": (257, 9, 7168, 256), "glm5": (257, 9, 6144, 2048), "kimik2": (384, 8, 7168, 256),
              "minimax_m25": (256, 8, 3072, 256), "qwen3_5_397b": (512, 10, 4096, 256)}
REF_MOE = {
    "deepseek": REF_MOE_STAGES,
    # aiter/configs/model_configs/glm5_fp4_tuned_fmoe.csv:2,6,9,12,14
    "glm5": {1: (23.1763, 16.8433), 16: (233.4281, 127.2874), 128: (513.8856, 276.6438),
             1024: (544.8517, 320.5397), 4096: (978.5945, 784.0105)},
    # aiter/configs/model_configs/kimik2_fp4_tuned_fmoe.csv:2,6,9,12,14
    "kimik2": {1: (13.6475, 7.7145), 16: (35.9287, 23.6549), 128: (108.3724, 66.6968),
               1024: (121.0563, 106.3806), 4096: (158.9084, 270.351)},
    # aiter/configs/model_configs/minimax_m25_fp4_tuned_fmoe.csv:2,6,9,12,14
    "minimax_m25": {1: (12.6929, 6.4582), 16: (19.2822, 15.3136), 128: (41.3453, 26.5566),
                    1024: (45.8141, 47.6451), 4096: (82.4129, 126.4326)},
    # aiter/configs/model_configs/qwen3_5_397b_fp4_tuned_fmoe.csv:2,6,9,12,14
    "qwen3_5_397b": {1: (19.3721, 0.0), 16: (55.31, 0.0), 128: (87.4931, 53.1125), 1024: (110.6725, 81.2088),
                     4096: (149.0609, 201.2182)},
}


def fused_moe_module():
    """The aiter_amd.fused_moe module (the package attribute of that name is
    the fused_moe function)."""
    import importlib

    return importlib.import_module("aiter_amd.fused_moe")


def _moe_stage_times(aiter_amd, x, w1, w2, w1s, w2s, tw, ti, E, topk, dim, inter, ref=None):
    """Each launch group of fused_moe timed on its own (graph-replayed, inputs
    from an eager run of the steps before it): the routing sort, the sorted
    activation quant, stage 1 with its fused output quant (and its split-K
    reduce) and stage 2 (with moe_sum when the per-pair rows are reduced by
    slot), for a like-for-like comparison with the reference's tuned us1 /
    us2 (stage kernels only; its decode rows' stage 1 also quantises its
    output, the "_fp4" kernels of dsv3_fp4_tuned_fmoe.csv)."""
    from aiter_amd import dtypes

    FM = fused_moe_module()

    m = x.shape[0]
    bm = FM.get_block_size_M(m, topk, E, inter)
    reduce = FM._use_reduce(m, topk)
    qt = int(aiter_amd.QuantType.per_1x32)
    sort = lambda: FM.moe_sorting(ti, tw, E, dim, torch.bfloat16, bm, None, None, 0, accumulate=not reduce)
    sids, sw, seids, nv, moe_buf = sort()
    q1 = lambda: FM.fused_dynamic_mx_quant_moe_sort(x, sids, nv, m, topk, bm, dtypes.fp4x2, sorted_weights=sw)
    a1, a1s = q1()
    # stage 1 with its output quantised in the same launch (the flow fused_moe
    # takes here; the reference's fuse_quant "fp4" stage 1)
    s1 = lambda: FM.ck_moe_stage1_fuse_quant(a1, w1, sids, seids, nv, m, topk, bm, w1s, a1s, None, sw,
                                             int(FM.ActivationType.Silu))
    a2q, a2s = s1()
    if FM.can_sort_quant(x, ti):
        # decode: fused_moe sorts and quantises the tokens in one launch
        sq = lambda: FM.moe_sorting_mx_quant(ti, tw, x, E, bm, accumulate=not reduce)
        sq()
        res = {"sort_us": time_graph(sq, 10, 2), "quant1_us": 0.0, "sort_quant_fused": True}
    else:
        res = {"sort_us": time_graph(sort, 10, 2), "quant1_us": time_graph(q1, 10, 2), "sort_quant_fused": False}
    res.update({"stage1_us": time_graph(s1, 10, 2), "quant2_us": 0.0})
    if reduce:
        per_pair = torch.empty((m, topk, dim), dtype=torch.bfloat16, device=x.device)
        s2 = lambda: FM.ck_moe_stage2(a2q, w1, w2, sids, seids, nv, per_pair, topk, "", w2s, a2s, bm, sw, qt)
        s2()
        res["stage2_us"] = time_graph(s2, 10, 2)
        moe_out = torch.empty((m, dim), dtype=torch.bfloat16, device=x.device)   # moe_buf is empty here
        res["moe_sum_us"] = time_graph(lambda: FM.moe_sum(per_pair, moe_out), 10, 2)
    else:
        s2 = lambda: FM.ck_moe_stage2(a2q, w1, w2, sids, seids, nv, moe_buf, topk, "", w2s, a2s, bm, sw, qt)
        res["stage2_us"] = time_graph(s2, 10, 2)
        res["moe_sum_us"] = 0.0
    res = {k: (round(v * 1e6, 1) if isinstance(v, float) else v) for k, v in res.items()}
    res["stages_us"] = round(res["stage1_us"] + res["stage2_us"] + res["moe_sum_us"], 1)
    ref = REF_MOE_STAGES if ref is None else ref
    if m in ref:
        r1, r2 = ref[m]
        res["ref_stage1_us"], res["ref_stage2_us"] = r1, r2
        res["stages_vs_ref"] = round((r1 + r2) / res["stages_us"], 3)
    return res


def bf16_plumbing(dev):
    """A[128,4096] x B[4096,4096]^T bf16 from N(0,1) with
    seed 0.  The reference's CPU torch path (F.linear in bf16, and the fp32
    reference), median of 5 runs after 2 warm-ups on all host threads, next
    to the same GEMM on the GPU through gemm_a16w16 and its max error."""
    import platform

    import aiter_amd

    g = torch.Generator().manual_seed(0)
    a = torch.randn(128, 4096, generator=g).to(torch.bfloat16)
    b = torch.randn(4096, 4096, generator=g).to(torch.bfloat16)
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)

    def med(fn):
        for _ in range(2):
            fn()
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[2]

    t_bf16 = med(lambda: torch.nn.functional.linear(a, b))
    ref = (a.float() @ b.float().T)
    t_f32 = med(lambda: a.float() @ b.float().T)
    ad, bd = a.to(dev), b.to(dev)
    got = aiter_amd.gemm_a16w16(ad, bd).float().cpu()
    t_gpu = time_graph(lambda: aiter_amd.gemm_a16w16(ad, bd), 20, 5)
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        cpu_model = platform.processor() or "unknown"
    return {"cpu_bf16_linear_ms": round(t_bf16 * 1e3, 2), "cpu_f32_ref_ms": round(t_f32 * 1e3, 2),
            "cpu_threads": threads, "cpu_model": cpu_model, "gpu_us": round(t_gpu * 1e6, 2),
            "max_abs_err_vs_f32": round(float((got - ref).abs().max()), 4),
            "frac_within_1e-2": round(float(((got - ref.bfloat16().float()).abs()
                                            <= 1e-2 + 1e-2 * ref.bfloat16().float().abs()).float().mean()), 6)}


def cpu_threads():
    """Host threads the CPU baseline uses: the box's CPU share
    (OMP_NUM_THREADS when set, as on the GPU boxes), else every CPU."""
    env = os.environ.get("OMP_NUM_THREADS")
    return max(1, int(env)) if env and env.isdigit() else (os.cpu_count() or 1)


def cpu_baseline():
    """The reference's CPU torch path on the headline problem itself
    ``run_torch`` of op_tests/test_gemm_a4w4.py:23-39
    restated in oracle/torch_ref.py -- dequantise the MXFP4 A and B of
    M = N = K = 8192 to f32, one f32 ``torch.mm``, cast to bf16 -- on the
    host threads, 2 warm-ups then 1 timed run (the problem is above 100
    GFLOP).  ``value`` is the whole path's TFLOP/s; the dequantisation and
    the matmul are also timed separately."""
    import platform

    from oracle import torch_ref as T

    threads = cpu_threads()
    torch.set_num_threads(threads)
    m = n = k = 8192
    g = torch.Generator().manual_seed(0)
    # quantised operands of the headline shape (random e2m1 bytes, e8m0 near 2^0)
    aq = torch.randint(0, 256, (m, k // 2), dtype=torch.uint8, generator=g)
    bq = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, generator=g)
    asc = torch.randint(120, 134, (m, k // 32), dtype=torch.uint8, generator=g)
    bsc = torch.randint(120, 134, (n, k // 32), dtype=torch.uint8, generator=g)
    for _ in range(2):
        T.run_torch_a4w4(aq, bq, asc, bsc)
    tm = {}
    t0 = time.perf_counter()
    T.run_torch_a4w4(aq, bq, asc, bsc, timings=tm)
    total = time.perf_counter() - t0
    flop = 2.0 * m * n * k
    cpu_model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(flop / total / 1e12, 5), "unit": "TFLOP/s", "cores": int(torch.get_num_threads()),
            "kind": "port",
            "sample": f"the full M=N=K=8192 A4W4 problem: dequantise A and B to f32 ({tm['dequant_s']:.2f} s) + "
                      f"torch.mm f32 ({tm['mm_s']:.2f} s) + bf16 cast, {total:.2f} s, 1 timed run after 2 warm-ups",
            "dequant_s": round(tm["dequant_s"], 3), "mm_s": round(tm["mm_s"], 3),
            "mm_TFLOPs": round(flop / tm["mm_s"] / 1e12, 4), "cpu_model": cpu_model,
            "torch": torch.__version__}


def profile_workload(dev, name):
    """Launches for the rocprofv3 runs behind profiles/ (kernel trace, FETCH_SIZE,
    WRITE_SIZE, MFMA busy): three plain device copies of COPY_BYTES (the
    traffic counters' calibration), then three launches of workload ``name``,
    each after another copy (L2 and MALL start cold).  Every workload goes
    through the library's public entry point and its tuned dispatch."""
    import aiter_amd

    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    g = torch.Generator(device=dev).manual_seed(9)

    def bf16(r, c):
        return torch.randn((r, c), generator=g, device=dev).to(torch.bfloat16)

    if name == "a4w4_8192":
        aq, as_, bq, bs = quantised_operands(8192, 8192, 8192, 0, dev)
        fn = lambda: aiter_amd.gemm_a4w4(aq, bq, as_, bs)
    elif name in ("bf16_8192_bplain", "bf16_8192_bpre"):
        a, b = bf16(8192, 8192), bf16(8192, 8192)
        if name == "bf16_8192_bpre":
            b = aiter_amd.shuffle_weight(b)
        fn = lambda: aiter_amd.gemm_a16w16(a, b)
    elif name == "a8w4_4096x7168x16384":
        x, w = bf16(4096, 16384), bf16(7168, 16384)
        wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
        wq = aiter_amd.shuffle_weight(wq)
        xq, xs = aiter_amd.dynamic_mxfp8_quant(x, shuffle=True)
        fn = lambda: aiter_amd.gemm_a8w4_mxfp8(xq, wq, xs, ws, a_preshuffle=False)
    elif name == "quant_mxfp4_8192":
        x = bf16(8192, 8192)
        fn = lambda: aiter_amd.dynamic_mxfp4_quant(x, shuffle=True)
    elif name == "a4w4_splitk_256x14336x4096":
        aq, as_, bq, bs = quantised_operands(256, 14336, 4096, 0, dev)
        fn = lambda: aiter_amd.gemm_a4w4(aq, bq, as_, bs)
    elif name == "bf16_8192x8192x28672":
        a, b = bf16(8192, 28672), bf16(8192, 28672)
        fn = lambda: aiter_amd.gemm_a16w16(a, b)
    elif name == "bf16_256x8192x28672":
        a, b = bf16(256, 28672), bf16(8192, 28672)
        fn = lambda: aiter_amd.gemm_a16w16(a, b)
    elif name == "bf16_32x7168x2048":
        a, b = bf16(32, 2048), bf16(7168, 2048)
        fn = lambda: aiter_amd.gemm_a16w16(a, b)
    elif name == "fused_rms_mxfp4_8192":
        x, w = bf16(8192, 8192), bf16(1, 8192).view(-1)
        fn = lambda: aiter_amd.fused_rms_mxfp4_quant(x, w, 1e-6, shuffle=True)
    elif name.startswith("moe_deepseek_"):
        # fused_moe at the DeepSeek shape with "moe_deepseek_<tokens>" tokens
        m = int(name.rsplit("_", 1)[1])
        E, topk, dim, inter = 257, 9, 7168, 256
        w1 = aiter_amd.shuffle_weight(torch.randint(0, 256, (E * 2 * inter, dim // 2), dtype=torch.uint8,
                                                    device=dev, generator=g)).view(E, 2 * inter, dim // 2)
        w2 = aiter_amd.shuffle_weight(torch.randint(0, 256, (E * dim, inter // 2), dtype=torch.uint8, device=dev,
                                                    generator=g)).view(E, dim, inter // 2)
        w1s = aiter_amd.shuffle_scale(torch.randint(119, 123, (E * 2 * inter, dim // 32), dtype=torch.uint8,
                                                    device=dev, generator=g))
        w2s = aiter_amd.shuffle_scale(torch.randint(119, 123, (E * dim, inter // 32), dtype=torch.uint8, device=dev,
                                                    generator=g))
        x = bf16(m, dim)
        tw, ti = torch.topk(torch.softmax(torch.randn(m, E, device=dev, generator=g), -1), topk, -1)
        tw, ti = (tw / tw.sum(-1, keepdim=True)).float(), ti.to(torch.int32)
        fn = lambda: aiter_amd.fused_moe(x, w1, w2, tw, ti, quant_type=aiter_amd.QuantType.per_1x32, w1_scale=w1s,
                                         w2_scale=w2s)
    elif _shape_workload(name):
        # "<a4w4|bf16|a8w4>_<M>x<N>x<K>": that GEMM through its public entry
        fam, (m, n, k) = _shape_workload(name)
        if fam == "a4w4":
            aq, as_, bq, bs = quantised_operands(m, n, k, 0, dev)
            fn = lambda: aiter_amd.gemm_a4w4(aq, bq, as_, bs)
        elif fam == "a8w4":
            x, w = bf16(m, k), bf16(n, k)
            wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
            wq = aiter_amd.shuffle_weight(wq)
            xq, xs = aiter_amd.dynamic_mxfp8_quant(x, shuffle=True)
            fn = lambda: aiter_amd.gemm_a8w4_mxfp8(xq, wq, xs, ws, a_preshuffle=False)
        else:
            a, b = bf16(m, k), bf16(n, k)
            ot = torch.float32 if fam == "bf16f32" else None
            fn = lambda: aiter_amd.gemm_a16w16(a, b, otype=ot)
    else:
        raise SystemExit(f"unknown workload {name}")
    fn()
    for _ in range(3):
        dst.copy_(src)
    for _ in range(3):
        dst.copy_(src)
        fn()
    torch.cuda.synchronize()
    log(f"profile workload done: copy {COPY_BYTES} B x6, {name} x3 (+1 warm-up call)")


def _shape_workload(name):
    """("a4w4" | "bf16" | "bf16f32" | "a8w4", (M, N, K)) for a workload named
    "<family>_<M>x<N>x<K>" (bf16f32: bf16 inputs, f32 output), else None."""
    fam, _, dims = name.partition("_")
    parts = dims.split("x")
    if fam not in ("a4w4", "bf16", "bf16f32", "a8w4") or len(parts) != 3 or not all(p.isdigit() for p in parts):
        return None
    return fam, tuple(int(p) for p in parts)


def traffic_from_profiles():
    p = os.path.join(ROOT, "profiles", "a4w4_8192_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--moe", action="store_true", help="only the fused-MoE workloads (for profiling)")
    ap.add_argument("--moe-models", action="store_true",
                    help="fused MoE at each MOE_MODELS shape against the reference's tuned stage times")
    ap.add_argument("--decode", action="store_true", help="only the decode workloads (configs[1] and configs[4])")
    ap.add_argument("--sweep", action="store_true", help="only the prefill sweep (configs[4]) and configs[3]")
    ap.add_argument("--cpu", action="store_true", help="only the CPU baseline")
    ap.add_argument("--workload", default=None,
                    help="only the launches of one profiled workload (see profile_workload)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    import aiter_amd  # noqa: F401  (fails loudly if the HIP library is missing)
    if args.workload:
        profile_workload(dev, args.workload)
        return
    if args.moe:
        print(json.dumps({"fused_moe_a4w4_deepseek": bench_moe(dev)}), flush=True)
        return
    if args.moe_models:
        res = {}
        for name in MOE_MODELS:
            res[name] = bench_moe(dev, model=name)
            torch.cuda.empty_cache()
        print(json.dumps({"fused_moe_models": res}), flush=True)
        return
    if args.decode:
        print(json.dumps({"decode": bench_decode(dev), "decode_sweep": bench_decode_sweep(dev)}), flush=True)
        return
    if args.sweep:
        print(json.dumps({"prefill_sweep": bench_prefill_sweep(dev), "a8w4_mxfp8": bench_a8w4(dev)}), flush=True)
        return
    if args.cpu:
        print(json.dumps({"cpu_baseline": cpu_baseline()}), flush=True)
        return

    log("prefill A4W4 8192^3")
    sec, tflops, kname = bench_prefill(args.steps, args.warmup, dev)
    log(f"prefill: {sec*1e6:.1f} us/step, {tflops:.0f} TFLOP/s ({kname or 'heuristic'})")
    decode = [] if args.quick else bench_decode(dev)
    sweep = [] if args.quick else bench_decode_sweep(dev)
    prefill_sweep = [] if args.quick else bench_prefill_sweep(dev)
    a8w4 = [] if args.quick else bench_a8w4(dev)
    extra = {} if args.quick else bench_extra(dev)
    cpu = None if (args.no_cpu or args.quick) else cpu_baseline()
    m = n = k = 8192
    line = {
        "metric": "TFLOP/s and % dense MXFP4/bf16 peak (M=8192); HBM GB/s % peak at M<=32",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tflops / REF_A4W4_8192, 4),
        "dtype": "mxfp4",
        "data": "synthetic",
        "config": {"workload": "A4W4 MXFP4xMXFP4 GEMM, M=N=K=8192, preshuffled B, e8m0 per-1x32 scales, bf16 out "
                               "(BASELINE configs[2])", "M": m, "N": n, "K": k, "kernel": kname or "heuristic"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK_MXFP4, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_MXFP4, 4), "traffic": traffic_from_profiles()},
        "cpu_baseline": cpu,
        "decode": decode,
        "decode_sweep": sweep,
        "prefill_sweep": prefill_sweep,
        "a8w4_mxfp8": a8w4,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
