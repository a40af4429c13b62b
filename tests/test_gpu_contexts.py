"""GPU checks of the context calls under wgblas's device handling, through
the C ABI: init({benchmark: true}) opens a second wgb_ctx on the same device
with per-call timing on (src/init.mjs:31-108, gpuTimeMs from
src/util/benchmark.mjs:14-103), and cleanup(device) destroys one context while
the others keep working (src/init.mjs:110-131). The JavaScript layer's side
of the same handling (the cache keyed by options, which device cleanup(one)
releases) is checked on the CPU against a host-memory stand-in addon
(tests/js/devices_cpu.mjs).
"""
import numpy as np
import pytest

from tests.helpers import bits_equal

pytestmark = pytest.mark.gpu


def test_second_context_timing_and_release(ctx):
    from wgblas_amd import Context
    from wgblas_amd.native import WgblasError

    n, n2 = 1024, 2048
    A = ctx.empty(n2 * n2, np.float32)
    B = ctx.empty(n2 * n2, np.float32)
    C1, C2, C3 = (ctx.empty(n2 * n2, np.float32) for _ in range(3))
    ctx.fill_uniform(A, -1, 1, 81)
    ctx.fill_uniform(B, -1, 1, 82)
    ctx.synchronize()  # the other context's stream reads them next
    print("contexts case: second context with timing", flush=True)
    bench = Context(0)
    try:
        assert bench.name()[1].startswith(ctx.name()[1].split(":")[0])
        # untimed first calls: a kernel's first launch in the process loads
        # its code object, which a timed call would include
        bench.sgemm(0, 1, n, n, n, 1.0, A, n, B, n, 0.0, C2, n)
        bench.sgemm(0, 1, n2, n2, n2, 1.0, A, n2, B, n2, 0.0, C3, n2)
        bench.set_timing(True)
        with pytest.raises(WgblasError, match="no timed call"):
            bench.last_time_ms()
        bench.sgemm(0, 1, n, n, n, 1.0, A, n, B, n, 0.0, C2, n)
        small = bench.last_time_ms()
        bench.sgemm(0, 1, n2, n2, n2, 1.0, A, n2, B, n2, 0.0, C3, n2)
        big = bench.last_time_ms()
        # the events bracket the call's own kernels: eight times the flops
        # take longer, and neither time is zero or absurd
        assert 0.0 < small < big < 1000.0, (small, big)
        bench.synchronize()  # C2 / C3 are read on ctx's stream next
        # the untimed context has no timed call to report
        ctx.sgemm(0, 1, n, n, n, 1.0, A, n, B, n, 0.0, C1, n)
        with pytest.raises(WgblasError, match="no timed call"):
            ctx.last_time_ms()
        got1, got2 = C1.to_host()[: n * n], C2.to_host()[: n * n]
        assert bits_equal(got1, got2), "two contexts, same inputs, different bits"
    finally:
        bench.close()
    # cleanup of one device: the other context still computes, bit for bit
    print("contexts case: remaining context after the other was destroyed", flush=True)
    ctx.sgemm(0, 1, n, n, n, 1.0, A, n, B, n, 0.0, C3, n)
    assert bits_equal(C3.to_host()[: n * n], got1)
    # and a fresh context opened afterwards works too
    with Context(0) as again:
        again.sgemm(0, 1, n, n, n, 1.0, A, n, B, n, 0.0, C2, n)
        again.synchronize()
    assert bits_equal(C2.to_host()[: n * n], got1)
    for x in (A, B, C1, C2, C3):
        x.free()


def test_timing_switched_off_and_on(ctx):
    from wgblas_amd.native import WgblasError

    n = 512
    X = ctx.empty(3 * n * n, np.float32)
    ctx.fill_uniform(X, -1, 1, 83)
    try:
        ctx.set_timing(True)
        ctx.sgemm(0, 0, n, n, n, 1.0, X.offset(0), n, X.offset(n * n), n, 0.0, X.offset(2 * n * n), n)
        assert ctx.last_time_ms() > 0.0
        # switching timing on again forgets the last timed call
        ctx.set_timing(True)
        with pytest.raises(WgblasError, match="no timed call"):
            ctx.last_time_ms()
        ctx.set_timing(False)
        ctx.sgemm(0, 0, n, n, n, 1.0, X.offset(0), n, X.offset(n * n), n, 0.0, X.offset(2 * n * n), n)
        with pytest.raises(WgblasError, match="no timed call"):
            ctx.last_time_ms()
    finally:
        ctx.set_timing(False)
        ctx.synchronize()
        X.free()
