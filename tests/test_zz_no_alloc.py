"""GPU parity of wgb_sgemm_noalloc, the allocation-free sgemm entry point.

It runs wgb_sgemm's launches with the split-k partials in the library's fixed
per-GPU array instead of the context's hipMalloc'd workspace, so on the same
inputs it must return wgb_sgemm's bits exactly. The shapes put the launch on
the split-k path on an MI355X (256 CUs, two resident 128-tiles per CU, 512
slots: a round of whole tiles, then a tail at most half a round):
  * 3072 x 4096 x 1024: 768 tiles, the last 256 in 2 k-slices each, 512
    slices = the whole 32 MiB array;
  * 3071 x 3073 x 1777, ldc padded: 600 tiles, the last 88 in 5 slices, edge
    tiles and a partial k-tile in a slice;
  * 2944 x 2944 x 2048: 529 tiles, the last 17 in 16 k-slices each (17 MiB);
  * 2900 x 2950 x 1500, ldc padded, beta = 1: 552 tiles, the last 40 in 10
    slices.
Each case is two calls in a row on the one array, the second with a smaller
input, so the second call runs over whatever the first left in the array.
Every result is also checked on sampled columns against a float64 product
under the reference's forward-error bound (tests/sgemm/helpers.js:1-57), and
C's ld padding is bit-checked. On a fresh context, repeated split-k calls
leave the device's free memory (hipMemGetInfo) unchanged, while wgb_sgemm's
first split-k call on that context lowers it by its workspace.
"""
import ctypes

import numpy as np
import pytest

from tests.helpers import EPS32

pytestmark = pytest.mark.gpu


def _stored_rows(trans, rows, cols):
    """(rows, cols) of the column-major array holding op(X) = rows x cols."""
    return (cols, rows) if trans else (rows, cols)


def _make(ctx, ta, tb, m, n, k, ldc, seed):
    ar, ac = _stored_rows(ta, m, k)
    br, bc = _stored_rows(tb, k, n)
    A = ctx.empty(ac * ar, np.float32)
    B = ctx.empty(bc * br, np.float32)
    C0 = ctx.empty(n * ldc, np.float32)
    ctx.fill_uniform(A, -1, 1, seed)
    ctx.fill_uniform(B, -1, 1, seed + 1)
    ctx.fill_uniform(C0, -1, 1, seed + 2)
    return A, ar, B, br, C0


def _op(host, trans, rows, cols, ld):
    """op(X) as a dense float64 rows x cols array from column-major storage."""
    if trans:
        # stored cols x rows: stored column j is row j of op(X)
        return host.reshape(rows, ld)[:, :cols].astype(np.float64)
    return host.reshape(cols, ld)[:, :rows].T.astype(np.float64)


def _run_pair(ctx, ta, tb, m, n, k, alpha, beta, ldc, seed):
    A, lda, B, ldb, C0 = _make(ctx, ta, tb, m, n, k, ldc, seed)
    c_ref = ctx.empty(n * ldc, np.float32)
    c_new = ctx.empty(n * ldc, np.float32)
    try:
        ctx.synchronize()
        cin = C0.to_host()
        ctx.h2d(c_ref.ptr, cin)
        ctx.h2d(c_new.ptr, cin)
        ctx.sgemm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, c_ref, ldc)
        ctx.sgemm_noalloc(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, c_new, ldc)
        ctx.synchronize()
        got_ref, got_new = c_ref.to_host(), c_new.to_host()
        # the same launches on the same inputs: the same bits
        assert np.array_equal(got_ref.view(np.uint32), got_new.view(np.uint32)), \
            f"noalloc differs from wgb_sgemm at {m}x{n}x{k} ta={ta} tb={tb}"
        # ld padding of C untouched
        pad = np.ones((n, ldc), bool)
        pad[:, :m] = False
        assert np.array_equal(got_new.reshape(n, ldc)[pad].view(np.uint32),
                              cin.reshape(n, ldc)[pad].view(np.uint32))
        # sampled columns against float64 under the reference's bound
        ah = A.to_host()
        bh = B.to_host()
        opA = _op(ah, ta, m, k, lda)
        opB = _op(bh, tb, k, n, ldb)
        rng = np.random.default_rng(seed)
        cols = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 24)]))
        ref = alpha * (opA @ opB[:, cols]) + beta * cin.reshape(n, ldc)[cols, :m].T.astype(np.float64)
        absdot = np.abs(opA) @ np.abs(opB[:, cols])
        bound = EPS32 * ((k + 1) * abs(alpha) * absdot
                         + abs(beta) * np.abs(cin.reshape(n, ldc)[cols, :m].T))
        got = got_new.reshape(n, ldc)[cols, :m].T.astype(np.float64)
        assert np.all(np.abs(got - ref) <= bound)
    finally:
        for x in (A, B, C0, c_ref, c_new):
            x.free()


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_noalloc_matches_sgemm_two_calls(ctx, ta, tb):
    # first call: the whole array (512 slices of 64 KiB); second, smaller:
    # 440 slices with edge tiles and a partial k-tile
    for (m, n, k, ldc, seed) in [(3072, 4096, 1024, 3072, 31), (3071, 3073, 1777, 3072, 32)]:
        print(f"noalloc case ta={ta} tb={tb} {m}x{n}x{k}", flush=True)
        _run_pair(ctx, ta, tb, m, n, k, 1.5, 0.5, ldc, seed)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_noalloc_tail_split_then_ragged(ctx, ta, tb):
    # 529 tiles (17 tail tiles in 16 slices), then a smaller ragged problem
    # with a padded ldc, beta = 1 and a partial k-tile (40 tail tiles in 10)
    print(f"noalloc case ta={ta} tb={tb} 2944^2x2048 then 2900x2950x1500", flush=True)
    _run_pair(ctx, ta, tb, 2944, 2944, 2048, 1.0, 0.25, 2944, 33)
    _run_pair(ctx, ta, tb, 2900, 2950, 1500, -0.75, 1.0, 2901, 34)


def test_noalloc_paths_without_split(ctx):
    # the one-launch small kernel, and alpha = 0 (the scale kernel): no
    # workspace, still wgb_sgemm's results
    print("noalloc case small kernel 300x200x100 and alpha = 0", flush=True)
    _run_pair(ctx, 0, 0, 300, 200, 100, 1.25, -0.5, 301, 35)
    _run_pair(ctx, 1, 1, 256, 128, 64, 0.0, 2.0, 256, 36)
    # the wide tier (whole 256 x 128 tiles filling a round of two blocks per
    # CU): no workspace either
    print("noalloc case wide tier 4096x4096x1024", flush=True)
    _run_pair(ctx, 1, 0, 4096, 4096, 1024, 1.5, 0.5, 4096, 37)


def _free_device_bytes():
    """hipMemGetInfo's free bytes on the current device (device 0)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_allocates_nothing_on_a_fresh_context():
    """The entry point called first on a new context (no wgb_sgemm before
    it, so no context workspace exists): once its array is loaded (the
    first call on the device), further split-k calls of two shapes change
    the device's free memory by nothing; wgb_sgemm's first split-k call on
    the same context then lowers it by its hipMalloc'd workspace, which
    shows the measure sees allocations of that size."""
    from wgblas_amd import Context

    print("noalloc case fresh context, free-memory check", flush=True)
    c = Context(0)
    bufs = []
    try:
        shapes = [(3072, 4096, 1024, 40), (2944, 2944, 2048, 41)]
        ops = []
        for (m, n, k, seed) in shapes:
            A, lda, B, ldb, C0 = _make(c, 0, 1, m, n, k, m, seed)
            bufs += [A, B, C0]
            ops.append((m, n, k, A, lda, B, ldb, C0))
        call = lambda op: c.sgemm_noalloc(0, 1, op[0], op[1], op[2], 1.0, op[3], op[4], op[5], op[6], 0.5,
                                          op[7], op[0])
        call(ops[0])  # loads the array on this device if no call has yet
        c.synchronize()
        before = _free_device_bytes()
        for _ in range(3):
            for op in ops:
                call(op)
        c.synchronize()
        after = _free_device_bytes()
        assert after == before, f"free device memory moved by {before - after} bytes across noalloc calls"
        m, n, k, A, lda, B, ldb, C0 = ops[0]
        c.sgemm(0, 1, m, n, k, 1.0, A, lda, B, ldb, 0.5, C0, m)
        c.synchronize()
        grown = _free_device_bytes()
        assert before - grown >= 16 << 20, \
            f"wgb_sgemm's workspace did not show in hipMemGetInfo ({before - grown} bytes)"
    finally:
        for x in bufs:
            x.free()
        c.close()


def test_noalloc_rejects_bad_arguments(ctx):
    from wgblas_amd.native import WgblasError

    A = ctx.empty(16, np.float32)
    try:
        with pytest.raises(WgblasError, match="lda"):
            ctx.sgemm_noalloc(0, 0, 4, 4, 4, 1.0, A, 3, A, 4, 0.0, A, 4)
        with pytest.raises(WgblasError, match="C is null"):
            ctx.sgemm_noalloc(0, 0, 4, 4, 4, 1.0, A, 4, A, 4, 0.0, None, 4)
    finally:
        A.free()
