#!/usr/bin/env python3
"""Throughput of wgblas's hot path on one MI355X, against its roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline ("step"): BASELINE config 3 — sgemm fp32 column-major
m = n = k = 8192 in all four (transA, transB) combinations, alpha = 1.5,
beta = 0.5; one step = the four GEMMs. `value` = 4 * 2mnk / step time.
Inputs: A, B, C drawn consecutively from one mulberry32(2) stream,
uniform[-1, 1) (wgblas's randomFloat32Array), generated and resident in HBM
before timing. Timing: HIP events recorded on the library's stream around
the K timed steps.

Also reported under "components", each timed the same way: sgemm 512^3
(config 1), the ragged sgemm 8191 x 8193 x 4097 with ld = 1 (mod 64)
(config 3), dgemm 4096^3 N/T alpha = beta = 1 (config 4), ssyrk lower
n = 8192, k = 4096, 10 chained resident calls (config 5), and sdot / sasum /
snrm2 / isamax at n = 2^28 plus the incx = 3, n = 2^26 variants (config 2),
sgemmtr on config 5's operands, ssyr2k / ssymm / strmm / strsm at order 8192
(strsm also 4096), dsyr2k / dsymm / dtrmm at order 4096, sgemv and dgemv
16384 x 16384 in both forms, sger / dger and ssyr / dsyr / ssyr2 / dsyr2 / ssymv /
dsymv (lower) at 16384, strmv / dtrmv (lower, N and T) at 16384, and ddot / dasum /
dnrm2 / idamax at n = 2^27
(the same bytes as config 2's fp32 vectors; uniform[-1, 1) inputs, seeds 1
and 2, as wgblas's randomFloat64Array).

`roofline` is for the headline kernel: algorithmic flops per launch (2mnk)
over the mean launch duration measured with events around each launch,
against the fp32 dense MFMA peak (157.3 TFLOP/s). `cpu_baseline` times the
oracle's restatement of the reference's per-element fp32 order on the host
(one thread) over a bounded sample of the same workload.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32 = 157.3e12
PEAK_FP64 = 78.6e12
PEAK_HBM = 8.0e12
METRIC = "sgemm/dgemm TFLOP/s + sdot/snrm2 GB/s on 1 MI355X, % of roofline"


class HipEvents:
    """hipEvent pairs on a given stream (libamdhip64 through ctypes)."""

    def __init__(self, stream):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)
        self.a, self.b = C.c_void_p(), C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(self.a)) == 0
        assert self.hip.hipEventCreate(C.byref(self.b)) == 0

    def start(self):
        assert self.hip.hipEventRecord(self.a, self.stream) == 0

    def stop_ms(self):
        assert self.hip.hipEventRecord(self.b, self.stream) == 0
        assert self.hip.hipEventSynchronize(self.b) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), self.a, self.b) == 0
        return ms.value


def timed(ctx, ev, fn, steps, warmup):
    """Runs fn() warmup + steps times; returns ms per step from events
    recorded on the library's stream around the timed steps."""
    for _ in range(warmup):
        fn()
    ctx.synchronize()
    ev.start()
    for _ in range(steps):
        fn()
    total = ev.stop_ms()
    return total / steps


def warm_up(ctx, fn, ms=30.0, max_calls=400):
    """Untimed calls of fn until about `ms` of wall time has passed: after
    the host-side set-up between workloads the clocks take some tens of
    milliseconds of load to settle (the first ragged 8191 x 8193 x 4097 NN
    calls ran 4.70, 4.45, 4.30, 4.17 ms, then 4.03 from the fifth on)."""
    t0 = time.perf_counter()
    for i in range(1, max_calls + 1):
        fn()
        if i % 4 == 0:
            ctx.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= ms:
                break
    ctx.synchronize()


def per_launch_ms(ctx, fn, reps, warm=False):
    """Mean duration of one library call measured by the library's events
    (wgb_set_timing), i.e. around that call's kernels only; with `warm`,
    after warm_up."""
    if warm:
        warm_up(ctx, fn)
    ctx.set_timing(True)
    acc = 0.0
    for _ in range(reps):
        fn()
        acc += ctx.last_time_ms()
    ctx.set_timing(False)
    return acc / reps


def rf(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
            "frac": achieved / peak, "traffic": traffic}


def traffic_entry(name):
    """(HBM bytes per launch, kernel) of workload `name`, measured with
    rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by a copy-kernel
    calibration) and recorded as `name = bytes  kernel` lines in
    profiles/traffic.txt; (None, None) when not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        if "=" not in line or line.lstrip().startswith("#"):
            continue
        key, rest = line.split("=", 1)
        if key.strip() != name:
            continue
        parts = rest.split(None, 1)
        try:
            return float(parts[0]), (parts[1].strip() if len(parts) > 1 else None)
        except (ValueError, IndexError):
            return None, None
    return None, None


def load_traffic(name):
    return traffic_entry(name)[0]


def headline_traffic():
    """Mean HBM bytes per launch over the four headline launches (the launches
    `roofline.achieved` averages) and, per layout, the bytes and the kernel
    that layout runs; (None, None) when any layout is unmeasured."""
    per = {lay: traffic_entry(f"sgemm_8192_{lay}") for lay in ("NN", "NT", "TN", "TT")}
    if any(v[0] is None for v in per.values()):
        return None, None
    mean = sum(v[0] for v in per.values()) / len(per)
    return mean, {lay: {"bytes": v[0], "kernel": v[1]} for lay, v in per.items()}


def bench_gemm_headline(ctx, ev, steps, warmup):
    from wgblas_amd import NO_TRANS, TRANS

    n = 8192
    buf = ctx.empty(3 * n * n, np.float32)
    ctx.fill_uniform(buf, -1.0, 1.0, 2)
    A, B, Cm = buf.offset(0), buf.offset(n * n), buf.offset(2 * n * n)
    combos = [(NO_TRANS, NO_TRANS), (NO_TRANS, TRANS), (TRANS, NO_TRANS), (TRANS, TRANS)]

    def step():
        for ta, tb in combos:
            ctx.sgemm(ta, tb, n, n, n, 1.5, A, n, B, n, 0.5, Cm, n)

    ms = timed(ctx, ev, step, steps, warmup)
    launch_ms = {}
    for ta, tb in combos:
        launch_ms["NT"[ta] + "NT"[tb]] = per_launch_ms(
            ctx, lambda: ctx.sgemm(ta, tb, n, n, n, 1.5, A, n, B, n, 0.5, Cm, n), max(3, steps))
    buf.free()
    flops = 2.0 * n * n * n
    mean_launch = sum(launch_ms.values()) / len(launch_ms)
    return ms, flops, launch_ms, mean_launch


def bench_components(ctx, ev, quick):
    from wgblas_amd import LOWER, NO_TRANS, TRANS

    comps = {}
    reps = 3 if quick else 10

    # config 1: sgemm 512^3 NN, alpha 1, beta 0; A then B from one seed-0
    # stream, C zero-initialised (the inputs test_gpu_fullsize.py checks)
    n = 512
    buf = ctx.empty(3 * n * n, np.float32)
    ctx.fill_uniform(buf, -1.0, 1.0, 0, n=2 * n * n)
    ctx.h2d(buf.offset(2 * n * n), np.zeros(n * n, np.float32))
    A, B, Cm = buf.offset(0), buf.offset(n * n), buf.offset(2 * n * n)
    f = lambda: ctx.sgemm(NO_TRANS, NO_TRANS, n, n, n, 1.0, A, n, B, n, 0.0, Cm, n)
    ms = per_launch_ms(ctx, f, 20, warm=True)
    comps["sgemm_512"] = {"ms": ms, "tflops": 2 * n ** 3 / ms / 1e9,
                          "frac_fp32_peak": 2 * n ** 3 / ms / 1e-3 / PEAK_FP32}
    buf.free()

    # config 3 ragged: 8191 x 8193 x 4097, ld = 1 (mod 64), all four layouts
    m, n, k = 8191, 8193, 4097
    ld = lambda r: ((r + 63) // 64) * 64 + 1
    fl = 2.0 * m * n * k
    per = {}
    for ta, tb in ((NO_TRANS, NO_TRANS), (NO_TRANS, TRANS), (TRANS, NO_TRANS), (TRANS, TRANS)):
        a_rows, a_cols = (k, m) if ta else (m, k)
        b_rows, b_cols = (n, k) if tb else (k, n)
        lda, ldb, ldc = ld(a_rows), ld(b_rows), ld(m)
        sa, sb, sc = lda * a_cols, ldb * b_cols, ldc * n
        buf = ctx.empty(sa + sb + sc, np.float32)
        ctx.fill_uniform(buf, -1.0, 1.0, 2)
        A, B, Cm = buf.offset(0), buf.offset(sa), buf.offset(sa + sb)
        f = lambda: ctx.sgemm(ta, tb, m, n, k, 1.5, A, lda, B, ldb, 0.5, Cm, ldc)
        ms = per_launch_ms(ctx, f, reps, warm=True)
        per["NT"[ta] + "NT"[tb]] = {"ms": ms, "tflops": fl / ms / 1e9, "ld": [lda, ldb, ldc]}
        buf.free()
    mean_ms = sum(v["ms"] for v in per.values()) / len(per)
    comps["sgemm_ragged_8191x8193x4097"] = {"ms": mean_ms, "tflops": fl / mean_ms / 1e9,
                                           "frac_fp32_peak": fl / mean_ms / 1e-3 / PEAK_FP32,
                                           "per_layout": per}

    # config 4: dgemm 4096^3, A N, B T, alpha = beta = 1, seed 3
    n = 4096
    buf = ctx.empty(3 * n * n, np.float64)
    ctx.fill_uniform(buf, -1.0, 1.0, 3)
    A, B, Cm = buf.offset(0), buf.offset(n * n), buf.offset(2 * n * n)
    fl = 2.0 * n ** 3
    per = {}
    # the configured NT first, then the other layouts on the same buffers
    for ta, tb in ((NO_TRANS, TRANS), (NO_TRANS, NO_TRANS), (TRANS, NO_TRANS), (TRANS, TRANS)):
        f = lambda: ctx.dgemm(ta, tb, n, n, n, 1.0, A, n, B, n, 1.0, Cm, n)
        ms = per_launch_ms(ctx, f, reps, warm=True)
        per["NT"[ta] + "NT"[tb]] = {"ms": ms, "tflops": fl / ms / 1e9}
    ms = per["NT"]["ms"]
    comps["dgemm_4096"] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp64_peak": fl / ms / 1e-3 / PEAK_FP64,
                           "traffic_bytes": load_traffic("dgemm_4096"), "per_layout": per}
    buf.free()

    # config 5: ssyrk lower, n = 8192, k = 4096, alpha 1, beta 0.25, 10 chained
    n, k = 8192, 4096
    dA = ctx.empty(n * k, np.float32)
    ctx.fill_normal(dA, 4)
    dC = ctx.empty(n * n, np.float32)
    ctx.fill_uniform(dC, -1.0, 1.0, 5)
    f = lambda: ctx.ssyrk(LOWER, NO_TRANS, n, k, 1.0, dA, n, 0.25, dC, n)
    warm_up(ctx, f)
    ev.start()
    for _ in range(10):
        f()
    ms = ev.stop_ms() / 10
    fl = float(n) * (n + 1) * k
    comps["ssyrk_8192x4096_x10"] = {"ms_per_call": ms, "tflops": fl / ms / 1e9,
                                    "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    # the same configuration through sgemmtr (lower, op(A) = A, op(B) = A^T)
    g = lambda: ctx.sgemmtr(LOWER, NO_TRANS, TRANS, n, n, k, 1.0, dA, n, dA, n, 0.25, dC, n)
    warm_up(ctx, g)
    ev.start()
    for _ in range(10):
        g()
    ms = ev.stop_ms() / 10
    comps["sgemmtr_8192x4096_x10"] = {"ms_per_call": ms, "tflops": fl / ms / 1e9,
                                      "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    # ssyr2k on the same shape: B = a second n x k operand (2 n(n+1) k flops,
    # wgblas's benchmarks/ssyr2k convention)
    dB = ctx.empty(n * k, np.float32)
    ctx.fill_normal(dB, 6)
    h = lambda: ctx.ssyr2k(LOWER, NO_TRANS, n, k, 1.0, dA, n, dB, n, 0.25, dC, n)
    ms = per_launch_ms(ctx, h, reps, warm=True)
    fl = 2.0 * n * (n + 1) * k
    comps["ssyr2k_8192x4096"] = {"ms": ms, "tflops": fl / ms / 1e9,
                                 "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    dA.free()
    dB.free()
    dC.free()
    comps.update(bench_level3(ctx, reps))
    comps.update(bench_level3_f64(ctx, reps))

    # sgemv, 16384 x 16384 (1 GiB of A, read once: the HBM roof), both forms
    n = 16384
    dA = ctx.empty(n * n, np.float32)
    ctx.fill_uniform(dA, -1.0, 1.0, 12)
    dx, dy = ctx.empty(n, np.float32), ctx.empty(n, np.float32)
    ctx.fill_uniform(dx, -1.0, 1.0, 13)
    ctx.fill_uniform(dy, -1.0, 1.0, 14)
    for t, tname in ((NO_TRANS, "N"), (TRANS, "T")):
        f = lambda: ctx.sgemv(t, n, n, 1.0, dA, n, dx, 1, 0.5, dy, 1)
        ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
        gbs = 4.0 * (n * n + 3 * n) / ms / 1e6
        comps[f"sgemv_{tname}_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
    dA.free()
    dx.free()
    dy.free()
    # dgemv on the same shape (2 GiB of A)
    dA = ctx.empty(n * n, np.float64)
    ctx.fill_uniform(dA, -1.0, 1.0, 12)
    dx, dy = ctx.empty(n, np.float64), ctx.empty(n, np.float64)
    ctx.fill_uniform(dx, -1.0, 1.0, 13)
    ctx.fill_uniform(dy, -1.0, 1.0, 14)
    for t, tname in ((NO_TRANS, "N"), (TRANS, "T")):
        f = lambda: ctx.dgemv(t, n, n, 1.0, dA, n, dx, 1, 0.5, dy, 1)
        ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
        gbs = 8.0 * (n * n + 3 * n) / ms / 1e6
        comps[f"dgemv_{tname}_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
    dA.free()
    dx.free()
    dy.free()

    # sger / dger on the same shape: A read and written once, alpha 1e-3
    for dt, name, es in ((np.float32, "sger", 4.0), (np.float64, "dger", 8.0)):
        dA = ctx.empty(n * n, dt)
        ctx.fill_uniform(dA, -1.0, 1.0, 15)
        dx, dy = ctx.empty(n, dt), ctx.empty(n, dt)
        ctx.fill_uniform(dx, -1.0, 1.0, 16)
        ctx.fill_uniform(dy, -1.0, 1.0, 17)
        fn = getattr(ctx, name)
        f = lambda: fn(n, n, 1e-3, dx, 1, dy, 1, dA, n)
        ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
        gbs = es * (2 * n * n + 2 * n) / ms / 1e6
        comps[f"{name}_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
        dA.free()
        dx.free()
        dy.free()

    # ssyr / dsyr, ssyr2 / dsyr2 (lower) on the same order: the triangle read
    # and written once
    for dt, pre, es in ((np.float32, "s", 4.0), (np.float64, "d", 8.0)):
        dA = ctx.empty(n * n, dt)
        ctx.fill_uniform(dA, -1.0, 1.0, 15)
        dx, dy = ctx.empty(n, dt), ctx.empty(n, dt)
        ctx.fill_uniform(dx, -1.0, 1.0, 16)
        ctx.fill_uniform(dy, -1.0, 1.0, 17)
        for name, f, vec in ((pre + "syr", lambda: getattr(ctx, pre + "syr")(LOWER, n, 1e-3, dx, 1, dA, n), 1),
                             (pre + "syr2", lambda: getattr(ctx, pre + "syr2")(LOWER, n, 1e-3, dx, 1, dy, 1,
                                                                             dA, n), 2)):
            ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
            gbs = es * (n * (n + 1) + vec * n) / ms / 1e6
            comps[f"{name}_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
        dA.free()
        dx.free()
        dy.free()

    # ssymv / dsymv (lower) on the same order: the triangle read once
    for dt, pre, es in ((np.float32, "s", 4.0), (np.float64, "d", 8.0)):
        dA = ctx.empty(n * n, dt)
        ctx.fill_uniform(dA, -1.0, 1.0, 18)
        dx, dy = ctx.empty(n, dt), ctx.empty(n, dt)
        ctx.fill_uniform(dx, -1.0, 1.0, 19)
        ctx.fill_uniform(dy, -1.0, 1.0, 20)
        f = lambda: getattr(ctx, pre + "symv")(LOWER, n, 1.0, dA, n, dx, 1, 0.5, dy, 1)
        ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
        gbs = es * (n * (n + 1) / 2 + 3 * n) / ms / 1e6
        comps[f"{pre}symv_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
        dA.free()
        dx.free()
        dy.free()

    # strmv / dtrmv (lower, both forms) on the same order: the triangle read
    # once, x read and y written
    for dt, pre, es in ((np.float32, "s", 4.0), (np.float64, "d", 8.0)):
        dA = ctx.empty(n * n, dt)
        ctx.fill_uniform(dA, -1.0, 1.0, 21)
        dx, dy = ctx.empty(n, dt), ctx.empty(n, dt)
        ctx.fill_uniform(dx, -1.0, 1.0, 22)
        for t, tname in ((0, "N"), (1, "T")):
            f = lambda: getattr(ctx, pre + "trmv")(LOWER, t, 0, n, dA, n, dx, 1, dy, 1)
            ms = per_launch_ms(ctx, f, 5 * reps, warm=True)
            gbs = es * (n * (n + 1) / 2 + 2 * n) / ms / 1e6
            comps[f"{pre}trmv_{tname}_16384"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
        dA.free()
        dx.free()
        dy.free()

    # config 2: reductions at n = 2^28 (normal seed 1 / 2, planted duplicate max)
    n = 1 << 28
    dx, dy = ctx.empty(n, np.float32), ctx.empty(n, np.float32)
    ctx.fill_normal(dx, 1)
    ctx.fill_normal(dy, 2)
    M = np.array([1e3, -1e3], np.float32)
    ctx.h2d(dx.offset(n // 3), M[:1])
    ctx.h2d(dx.offset(2 * n // 3), M[1:])
    out = ctx.empty(4, np.float32)
    iout = ctx.empty(1, np.int64)
    lreps = 20 if quick else 100
    red = {
        "sdot": (lambda inc, nn: ctx.sdot_dev(nn, dx, inc, dy, inc, out), 8),
        "sasum": (lambda inc, nn: ctx.sasum_dev(nn, dx, inc, out), 4),
        "snrm2": (lambda inc, nn: ctx.snrm2_dev(nn, dx, inc, out), 4),
        "isamax": (lambda inc, nn: ctx.isamax_dev(nn, dx, inc, iout), 4),
    }
    for name, (fn, bpe) in red.items():
        fn(1, n)
        ms = per_launch_ms(ctx, lambda: fn(1, n), lreps, warm=True)
        gbs = bpe * n / ms / 1e6
        comps[f"{name}_2^28"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM,
                                 "traffic_bytes": load_traffic(f"{name}_2^28")}
        ns = 1 << 26
        ms = per_launch_ms(ctx, lambda: fn(3, ns), lreps, warm=True)
        useful = bpe * ns / ms / 1e6
        comps[f"{name}_2^26_incx3"] = {"ms": ms, "GB/s_useful": useful,
                                       "GB/s_span": 3 * useful,
                                       "frac_hbm_peak_span": 3 * useful * 1e9 / PEAK_HBM}
    dx.free()
    dy.free()

    # the fp64 reductions over the same bytes: n = 2^27 doubles
    n = 1 << 27
    dx, dy = ctx.empty(n, np.float64), ctx.empty(n, np.float64)
    ctx.fill_uniform(dx, -1.0, 1.0, 1)
    ctx.fill_uniform(dy, -1.0, 1.0, 2)
    out = ctx.empty(4, np.float64)
    red = {
        "ddot": (lambda nn: ctx.ddot_dev(nn, dx, 1, dy, 1, out), 16),
        "dasum": (lambda nn: ctx.dasum_dev(nn, dx, 1, out), 8),
        "dnrm2": (lambda nn: ctx.dnrm2_dev(nn, dx, 1, out), 8),
        "idamax": (lambda nn: ctx.idamax_dev(nn, dx, 1, iout), 8),
    }
    for name, (fn, bpe) in red.items():
        fn(n)
        ms = per_launch_ms(ctx, lambda: fn(n), lreps, warm=True)
        gbs = bpe * n / ms / 1e6
        comps[f"{name}_2^27"] = {"ms": ms, "GB/s": gbs, "frac_hbm_peak": gbs * 1e9 / PEAK_HBM}
    dx.free()
    dy.free()
    return comps


def bench_level3(ctx, reps):
    """ssymm, strmm and strsm at order 8192 (left side, lower, no transpose),
    strsm also at 4096 (the top of wgblas's benchmarks/strsm sizes).
    `tflops` follows wgblas's benchmarks/<routine> flop conventions (ssymm
    2mn*order + 2mn, strmm 2mn*order + mn, strsm mn*order); `frac_fp32_peak`
    uses the arithmetic the routine must do (strmm: the triangle's
    mn*order)."""
    from wgblas_amd import LEFT, LOWER, NON_UNIT, NO_TRANS

    comps = {}
    n = 8192
    dA = ctx.empty(n * n, np.float32)
    dB = ctx.empty(n * n, np.float32)
    dC = ctx.empty(n * n, np.float32)
    ctx.fill_uniform(dA, -1.0, 1.0, 7)
    ctx.fill_uniform(dB, -1.0, 1.0, 8)
    ctx.fill_uniform(dC, -1.0, 1.0, 9)
    f = lambda: ctx.ssymm(LEFT, LOWER, n, n, 1.0, dA, n, dB, n, 0.5, dC, n)
    ms = per_launch_ms(ctx, f, reps, warm=True)
    fl = 2.0 * n * n * n + 2.0 * n * n
    comps["ssymm_8192"] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    f = lambda: ctx.strmm(LEFT, LOWER, NO_TRANS, NON_UNIT, n, n, 1.0, dA, n, dB, n)
    ms = per_launch_ms(ctx, f, reps, warm=True)
    fl_ref, fl = 2.0 * n * n * n + 1.0 * n * n, 1.0 * n * n * n
    comps["strmm_8192"] = {"ms": ms, "tflops": fl_ref / ms / 1e9, "tflops_triangle": fl / ms / 1e9,
                           "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    # strsm: a well-conditioned lower triangle (off-diagonals in [-1/n, 1/n),
    # diagonal 2, as wgblas's tests build it); B is re-filled before each
    # timed solve, outside the timed launch; untimed solves first (warm_up,
    # then two more on re-filled B)
    for order in (4096, 8192):
        ctx.fill_uniform(dA, -1.0 / order, 1.0 / order, 10)
        diag = np.full(1, 2.0, np.float32)
        for i in range(order):
            ctx.h2d(dA.offset(i * order + i), diag)
        fl = 1.0 * order * order * order
        solve = lambda: ctx.strsm(LEFT, LOWER, NO_TRANS, NON_UNIT, order, order, 1.0, dA, order,
                                  dB, order)
        warm_up(ctx, solve)
        times = []
        for it in range(2 + max(2, reps)):
            ctx.fill_uniform(dB, -1.0, 1.0, 11)
            t = per_launch_ms(ctx, solve, 1)
            if it >= 2:
                times.append(t)
        ms = sorted(times)[len(times) // 2]
        comps[f"strsm_{order}"] = {"ms": ms, "tflops": fl / ms / 1e9,
                                   "frac_fp32_peak": fl / ms / 1e-3 / PEAK_FP32}
    dA.free()
    dB.free()
    dC.free()
    return comps


def bench_level3_f64(ctx, reps):
    """dsyr2k (k = n), dsymm and dtrmm at order 4096 (dgemm's size; left
    side, lower, no transpose, alpha 1, beta 0: wgblas's benchmarks/<routine>
    defaults), with those benchmarks' flop conventions (dsyr2k 2n(n+1)k,
    dsymm 2mn*order + 2mn, dtrmm 2mn*order + mn); `frac_fp64_peak` uses the
    arithmetic the routine must do (dtrmm: the triangle's mn*order)."""
    from wgblas_amd import LEFT, LOWER, NON_UNIT, NO_TRANS

    comps = {}
    n = 4096
    dA, dB, dC = (ctx.empty(n * n, np.float64) for _ in range(3))
    ctx.fill_uniform(dA, -1.0, 1.0, 7)
    ctx.fill_uniform(dB, -1.0, 1.0, 8)
    ctx.fill_uniform(dC, -1.0, 1.0, 9)
    f = lambda: ctx.dsyr2k(LOWER, NO_TRANS, n, n, 1.0, dA, n, dB, n, 0.0, dC, n)
    ms = per_launch_ms(ctx, f, reps, warm=True)
    fl = 2.0 * n * (n + 1) * n
    comps["dsyr2k_4096"] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp64_peak": fl / ms / 1e-3 / PEAK_FP64}
    f = lambda: ctx.dsymm(LEFT, LOWER, n, n, 1.0, dA, n, dB, n, 0.0, dC, n)
    ms = per_launch_ms(ctx, f, reps, warm=True)
    fl = 2.0 * n * n * n + 2.0 * n * n
    comps["dsymm_4096"] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp64_peak": fl / ms / 1e-3 / PEAK_FP64}
    f = lambda: ctx.dtrmm(LEFT, LOWER, NO_TRANS, NON_UNIT, n, n, 1.0, dA, n, dB, n)
    ms = per_launch_ms(ctx, f, reps, warm=True)
    fl_ref, fl = 2.0 * n * n * n + 1.0 * n * n, 1.0 * n * n * n
    comps["dtrmm_4096"] = {"ms": ms, "tflops": fl_ref / ms / 1e9, "tflops_triangle": fl / ms / 1e9,
                           "frac_fp64_peak": fl / ms / 1e-3 / PEAK_FP64}
    dA.free()
    dB.free()
    dC.free()
    return comps


def run_only(ctx, name, reps, warm=False):
    """One workload alone, `reps` launches, for counter and kernel-trace runs
    (rocprofv3): copy (1 GiB device-to-device, the traffic calibration),
    sgemm_8192_{NN,NT,TN,TT}, config 3's ragged sgemm_ragged_{NN,NT,TN,TT},
    dgemm_4096_{NN,NT,TN,TT} (bare dgemm_4096: NT),
    ssyrk_8192, ssyr2k / ssymm / strmm / strsm at 8192 (strsm also 4096),
    dsyr2k / dsymm / dtrmm at 4096, sdot / sasum / snrm2 / isamax at
    n = 2^28. With `warm`, about 30 ms of the same calls run first (the
    clocks settle under load), so the traced launches match bench.py's."""
    from wgblas_amd import LOWER, NO_TRANS, TRANS

    def go(work, info):
        if warm:
            warm_up(ctx, work)
        for _ in range(reps):
            work()
        ctx.synchronize()
        return info

    def layout(lay):
        return (TRANS if lay[0] == "T" else NO_TRANS), (TRANS if lay[1] == "T" else NO_TRANS)

    if name == "copy":
        n = 1 << 28
        a, b = ctx.empty(n, np.float32), ctx.empty(n, np.float32)
        return go(lambda: ctx.lib.wgb_memcpy_d2d(ctx.handle, b.ptr, a.ptr, 4 * n),
                  {"bytes_read": 4 * n, "bytes_written": 4 * n})
    if name.startswith("sgemm_8192"):
        # one headline launch per call (bare name: NN)
        ta, tb = layout(name[len("sgemm_8192_"):] or "NN")
        n = 8192
        buf = ctx.empty(3 * n * n, np.float32)
        ctx.fill_uniform(buf, -1.0, 1.0, 2)
        return go(lambda: ctx.sgemm(ta, tb, n, n, n, 1.5, buf.offset(0), n, buf.offset(n * n), n, 0.5,
                                    buf.offset(2 * n * n), n), {"algorithmic_bytes": 4 * 4 * n * n})
    if name.startswith("sgemm_ragged"):
        # config 3's ragged case, one launch per call (bare name: NN)
        ta, tb = layout(name[len("sgemm_ragged_"):] or "NN")
        m, n, k = 8191, 8193, 4097
        ld = lambda r: ((r + 63) // 64) * 64 + 1
        a_rows, a_cols = (k, m) if ta else (m, k)
        b_rows, b_cols = (n, k) if tb else (k, n)
        lda, ldb, ldc = ld(a_rows), ld(b_rows), ld(m)
        sa, sb, sc = lda * a_cols, ldb * b_cols, ldc * n
        buf = ctx.empty(sa + sb + sc, np.float32)
        ctx.fill_uniform(buf, -1.0, 1.0, 2)
        return go(lambda: ctx.sgemm(ta, tb, m, n, k, 1.5, buf.offset(0), lda, buf.offset(sa), ldb, 0.5,
                                    buf.offset(sa + sb), ldc), {"algorithmic_bytes": 4 * (sa + sb + 2 * sc)})
    if name.startswith("dgemm_4096"):
        ta, tb = layout(name[len("dgemm_4096_"):] or "NT")
        n = 4096
        buf = ctx.empty(3 * n * n, np.float64)
        ctx.fill_uniform(buf, -1.0, 1.0, 3)
        return go(lambda: ctx.dgemm(ta, tb, n, n, n, 1.0, buf.offset(0), n, buf.offset(n * n), n, 1.0,
                                    buf.offset(2 * n * n), n), {"algorithmic_bytes": 8 * 4 * n * n})
    if name == "ssyrk_8192":
        n, k = 8192, 4096
        dA, dC = ctx.empty(n * k, np.float32), ctx.empty(n * n, np.float32)
        ctx.fill_normal(dA, 4)
        ctx.fill_uniform(dC, -1.0, 1.0, 5)
        return go(lambda: ctx.ssyrk(LOWER, NO_TRANS, n, k, 1.0, dA, n, 0.25, dC, n),
                  {"algorithmic_bytes": 4 * (n * k + n * (n + 1))})
    if name in ("ssyr2k_8192", "ssymm_8192", "strmm_8192", "strsm_8192", "strsm_4096"):
        from wgblas_amd import LEFT, NON_UNIT

        n = int(name.split("_")[1])
        dA, dB, dC = (ctx.empty(n * n, np.float32) for _ in range(3))
        ctx.fill_uniform(dA, -1.0 / n, 1.0 / n, 10)
        ctx.fill_uniform(dC, -1.0, 1.0, 9)
        diag = np.full(1, 2.0, np.float32)
        for i in range(n):
            ctx.h2d(dA.offset(i * n + i), diag)

        def work():
            ctx.fill_uniform(dB, -1.0, 1.0, 11)
            if name == "ssyr2k_8192":
                ctx.ssyr2k(LOWER, NO_TRANS, n, n // 2, 1.0, dA, n, dB, n, 0.25, dC, n)
            elif name == "ssymm_8192":
                ctx.ssymm(LEFT, LOWER, n, n, 1.0, dA, n, dB, n, 0.5, dC, n)
            elif name == "strmm_8192":
                ctx.strmm(LEFT, LOWER, NO_TRANS, NON_UNIT, n, n, 1.0, dA, n, dB, n)
            else:
                ctx.strsm(LEFT, LOWER, NO_TRANS, NON_UNIT, n, n, 1.0, dA, n, dB, n)

        return go(work, {"algorithmic_bytes": 4 * 3 * n * n})
    if name in ("dsyr2k_4096", "dsymm_4096", "dtrmm_4096"):
        from wgblas_amd import LEFT, NON_UNIT

        n = 4096
        dA, dB, dC = (ctx.empty(n * n, np.float64) for _ in range(3))
        ctx.fill_uniform(dA, -1.0, 1.0, 7)
        ctx.fill_uniform(dC, -1.0, 1.0, 9)

        def work():
            ctx.fill_uniform(dB, -1.0, 1.0, 8)
            if name == "dsyr2k_4096":
                ctx.dsyr2k(LOWER, NO_TRANS, n, n, 1.0, dA, n, dB, n, 0.0, dC, n)
            elif name == "dsymm_4096":
                ctx.dsymm(LEFT, LOWER, n, n, 1.0, dA, n, dB, n, 0.0, dC, n)
            else:
                ctx.dtrmm(LEFT, LOWER, NO_TRANS, NON_UNIT, n, n, 1.0, dA, n, dB, n)

        return go(work, {"algorithmic_bytes": 8 * 3 * n * n})
    n = 1 << 28
    dx, dy = ctx.empty(n, np.float32), ctx.empty(n, np.float32)
    ctx.fill_normal(dx, 1)
    ctx.fill_normal(dy, 2)
    out, iout = ctx.empty(4, np.float32), ctx.empty(1, np.int64)
    fns = {"sdot": lambda: ctx.sdot_dev(n, dx, 1, dy, 1, out), "sasum": lambda: ctx.sasum_dev(n, dx, 1, out),
           "snrm2": lambda: ctx.snrm2_dev(n, dx, 1, out), "isamax": lambda: ctx.isamax_dev(n, dx, 1, iout)}
    return go(fns[name], {"algorithmic_bytes": (8 if name == "sdot" else 4) * n})


def vendor_twin():
    """rocBLAS on the same workloads and inputs (wgblas_amd/lib/vendor_twin,
    run as a child process): {workload: {shape, ms, TFLOP/s | GB/s}}, or a
    note when the twin is not built. Context next to the components, not a
    parity check."""
    import subprocess

    exe = os.path.join(ROOT, "wgblas_amd", "lib", "vendor_twin")
    if not os.path.exists(exe):
        return {"note": "vendor_twin not built (python -m wgblas_amd.build)"}
    res = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=600)
    out = {}
    for ln in res.stdout.splitlines():
        try:
            rec = json.loads(ln)
        except ValueError:
            continue
        name = rec.pop("workload")
        rec.pop("library", None)
        out[name] = rec
    out["version"] = res.stderr.strip().splitlines()[-1] if res.stderr.strip() else "rocBLAS"
    if res.returncode != 0:
        out["error"] = f"exit {res.returncode}"
    return out


def roof_probe():
    """The roofs re-measured on this box (wgblas_amd/lib/roof_probe, run as a
    child process): HBM read and copy bandwidth, fp32 / fp64 MFMA issue
    rate. Context beside the published peaks that `roofline` uses."""
    import subprocess

    exe = os.path.join(ROOT, "wgblas_amd", "lib", "roof_probe")
    if not os.path.exists(exe):
        return {"note": "roof_probe not built (python -m wgblas_amd.build)"}
    res = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    out = {}
    for ln in res.stdout.splitlines():
        try:
            rec = json.loads(ln)
        except ValueError:
            continue
        out[rec.pop("probe")] = rec
    if res.returncode != 0:
        out["error"] = f"exit {res.returncode}: {res.stderr.strip()[-200:]}"
    return out


def reference_cpu_adapter_probe():
    """What this host offers for running the reference itself on a CPU
    WebGPU adapter (Dawn on Mesa lavapipe, the recipe of wgblas's
    .github/actions/lavapipe/action.yml): Node >= 22 (wgblas's package.json
    engines), the `webgpu` npm package (prebuilt Dawn) and a Vulkan ICD."""
    import shutil
    import subprocess

    info = {"node": None, "webgpu_package": False, "vulkan_icds": []}
    node = shutil.which("node")
    if node:
        r = subprocess.run([node, "--version"], capture_output=True, text=True, timeout=30)
        info["node"] = r.stdout.strip() or None
        r = subprocess.run([node, "-e", "require.resolve('webgpu')"], capture_output=True, text=True,
                           timeout=30)
        info["webgpu_package"] = r.returncode == 0
    for d in ("/usr/share/vulkan/icd.d", "/etc/vulkan/icd.d", "/usr/local/share/vulkan/icd.d"):
        if os.path.isdir(d):
            info["vulkan_icds"] += sorted(os.path.join(d, f) for f in os.listdir(d))
    major = None
    if info["node"] and info["node"].startswith("v"):
        try:
            major = int(info["node"][1:].split(".")[0])
        except ValueError:
            major = None
    missing = []
    if major is None or major < 22:
        missing.append(f"Node >= 22 (found {info['node']})")
    if not info["webgpu_package"]:
        missing.append("the webgpu npm package")
    if not info["vulkan_icds"]:
        missing.append("a Vulkan ICD (lavapipe)")
    info["runnable"] = not missing
    if missing:
        info["reason"] = "missing " + ", ".join(missing) + "; nothing can be installed (no network)"
    if not info["vulkan_icds"]:
        del info["vulkan_icds"]  # keeps the line's end short; `reason` names what is missing
    return info


def cpu_baseline(budget_s=4.0):
    """The oracle's fp32 restatement of the reference's per-element order
    (oracle/oracle.c orc_sgemm_wgsl) on the headline workload's inputs (A, B,
    C from one mulberry32(2) stream), transA = T, transB = N, alpha 1.5,
    beta 0.5: every host core the process may use runs its own 8-column
    chunks of C (ctypes releases the GIL), for `budget_s` seconds. A bounded
    sample, reported beside the reference's own CPU-adapter status."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import orc

    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    n, chunk = 8192, 8
    stream = orc.random_f32(3 * n * n, -1.0, 1.0, 2)
    A, B, C0 = stream[:n * n], stream[n * n:2 * n * n], stream[2 * n * n:]

    def worker(t):
        cols, c = 0, t * chunk
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s and c < n:
            orc.sgemm_wgsl(0, 1, 0, n, chunk, n, 1.5, A, n, B[c * n:(c + chunk) * n], n, 0.5,
                           C0[c * n:(c + chunk) * n], n)
            cols += chunk
            c += threads * chunk
        return cols

    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        cols = sum(ex.map(worker, range(threads)))
    wall = time.perf_counter() - t0
    flops = 2.0 * n * n * cols
    return {"value": flops / wall / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "host_cpus_usable": len(os.sched_getaffinity(0)),
            "sample": f"oracle orc_sgemm_wgsl (reference per-element fp32 order), transA=T transB=N, "
                      f"m=k=8192, {cols} columns of C over {threads} threads ({flops:.3g} flop in "
                      f"{wall:.1f} s wall)",
            "reference_cpu_adapter": reference_cpu_adapter_probe()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="fewer repetitions for the components")
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help="run one workload alone (copy, sgemm_8192_{NN,NT,TN,TT}, sgemm_ragged_{NN,NT,TN,TT}, "
                         "dgemm_4096[_{NN,NT,TN,TT}], ssyrk_8192, "
                         "ssyr2k_8192, ssymm_8192, strmm_8192, strsm_8192, strsm_4096, dsyr2k_4096, dsymm_4096, dtrmm_4096, "
                         "sdot, sasum, snrm2, "
                         "isamax) for counter and kernel-trace collection")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--warm", action="store_true",
                    help="with --only: about 30 ms of untimed calls before the reps")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the rocBLAS twin (wgblas_amd/lib/vendor_twin) of the components "
                         "and the roof probe (wgblas_amd/lib/roof_probe)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))

    from wgblas_amd import Context

    ctx = Context(0)
    if args.only:
        info = run_only(ctx, args.only, args.reps, args.warm)
        ctx.close()
        print(json.dumps({"only": args.only, "reps": args.reps, **info}))
        return 0
    ev = HipEvents(ctx.stream)
    name, arch = ctx.name()
    traffic, traffic_detail = headline_traffic()
    ms, flops, launch_ms, mean_launch = bench_gemm_headline(ctx, ev, args.steps, args.warmup)
    value = 4 * flops / (ms * 1e-3) / 1e12
    achieved = flops / (mean_launch * 1e-3) / 1e12
    comps = {} if args.no_components else bench_components(ctx, ev, args.quick)
    ctx.close()
    vendor = None if (args.no_vendor or args.no_components) else vendor_twin()
    roofs = None if (args.no_vendor or args.no_components) else roof_probe()
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (mulberry32 seeded uniform[-1,1), resident in HBM)",
        "config": {"workload": "sgemm fp32 column-major m=n=k=8192, transA/transB in {N,T}^2 "
                               "(4 GEMMs per step), alpha=1.5, beta=0.5, seed 2",
                   "m": 8192, "n": 8192, "k": 8192, "device": name, "arch": arch},
        "roofline": rf("mfma", achieved, PEAK_FP32 / 1e12, "TFLOP/s", traffic),
        "traffic_per_layout": traffic_detail,
        "sgemm_launch_ms": launch_ms,
        "components": comps,
    }
    if vendor is not None:
        line["vendor_rocblas"] = vendor
    if roofs is not None:
        line["roof_probe"] = roofs
    if rank == 0 and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    if comps:
        line["summary"] = summary(line)
    if rank == 0:
        print(json.dumps(line))
    return 0


def summary(line):
    """Every BASELINE configuration's figure in a few hundred bytes, the last
    key of the line (a reader that keeps only the end of the output still
    sees all of them): c1 sgemm 512^3 (us per call), c2 the reductions at
    2^28 (GB/s) and their incx = 3 forms at 2^26 (GB/s of span), c3 the
    8192^3 layouts and the ragged 8191x8193x4097 layouts (TFLOP/s), c4 dgemm
    4096^3 per layout (TFLOP/s), c5 ssyrk / sgemmtr 8192 k 4096 (TFLOP/s),
    and the level-3 callers as fractions of their peak."""
    c = line["components"]
    r1 = lambda x: round(x, 1)
    flops = 2.0 * 8192 ** 3
    s = {"c1_sgemm512_us": r1(c["sgemm_512"]["ms"] * 1e3)}
    red = ("sdot", "sasum", "snrm2", "isamax")
    s["c2_GBps"] = {r: round(c[f"{r}_2^28"]["GB/s"]) for r in red}
    s["c2_inc3_span_GBps"] = {r: round(c[f"{r}_2^26_incx3"]["GB/s_span"]) for r in red}
    c3 = {"mean": r1(line["value"])}
    c3.update({lay: r1(flops / ms / 1e9) for lay, ms in line["sgemm_launch_ms"].items()})
    s["c3_TF"] = c3
    s["c3_ragged_TF"] = {lay: r1(v["tflops"])
                         for lay, v in c["sgemm_ragged_8191x8193x4097"]["per_layout"].items()}
    s["c4_dgemm_TF"] = {lay: r1(v["tflops"]) for lay, v in c["dgemm_4096"]["per_layout"].items()}
    s["c5_TF"] = {"ssyrk": r1(c["ssyrk_8192x4096_x10"]["tflops"]),
                  "sgemmtr": r1(c["sgemmtr_8192x4096_x10"]["tflops"])}
    fr = {}
    for key, name in (("ssyr2k_8192x4096", "ssyr2k"), ("ssymm_8192", "ssymm"), ("strmm_8192", "strmm"),
                      ("strsm_4096", "strsm4k"), ("strsm_8192", "strsm8k"), ("dsyr2k_4096", "dsyr2k"),
                      ("dsymm_4096", "dsymm"), ("dtrmm_4096", "dtrmm")):
        if key in c:
            v = c[key]
            fr[name] = round(v.get("frac_fp32_peak", v.get("frac_fp64_peak", 0.0)), 3)
    s["l3_frac_of_peak"] = fr
    s["headline_frac"] = round(line["roofline"]["frac"], 3)
    return s


if __name__ == "__main__":
    sys.exit(main())
