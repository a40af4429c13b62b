"""GPU parity of dsyr2k, dsymm and dtrmm (native fp64 on the GEMM kernel)
through the C ABI, against the oracle's long-double restatements, under the
reference's own metrics with its double-double eps 2^-48:

  * dsyr2k (tests/dsyr2k/helpers.js): eps ((k+2)|alpha| d1 + (k+1)|alpha| d2
    + 2|beta||C_in|) on the triangle; the other triangle bit-identical.
  * dsymm (tests/dsymm/helpers.js): eps ((order+2)|alpha| sum|S B| + 3|beta||C_in|).
  * dtrmm (tests/dtrmm/helpers.js): eps (order+2) |alpha| sum|op(A) B|.

The scenarios follow tests/{dsyr2k,dsymm,dtrmm}/src/test.*.js: the edge-case
fixtures in both layouts, the multi-tile 150 / 400 paths, zero dimensions,
quick returns, ld padding, IEEE special values and alpha = 0. The reference's
double-double keeps f32's exponent range and pins that in its "f32 exponent
range" regressions; native fp64 keeps f64's, so here the same inputs (1e300,
1e-50, a result past 3.4e38) are checked against the oracle's f64-range
result instead.
"""
import itertools

import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS_DD, bits_equal
from tests.test_gpu_level3 import c_term, factor, outside, region

pytestmark = pytest.mark.gpu

F64 = np.float64


def up(ctx, a):
    a = np.asarray(a, F64)
    return ctx.upload(a if a.size else np.zeros(1, F64))


def at(n, i, j):
    """Row-major index of (i, j) in an n x n matrix (the reference's `at`)."""
    return i * n + j


def ieee_factor(got, ref, bound, idx):
    """NaN where the oracle has NaN, the oracle's infinities exactly, and the
    forward-error factor over the entries the oracle finds finite."""
    g = np.asarray(got, F64)[idx]
    r = np.asarray(ref, F64)[idx]
    assert np.array_equal(np.isnan(g), np.isnan(r))
    inf = np.isinf(r)
    assert np.array_equal(g[inf], r[inf])
    return factor(got, ref, bound, idx[np.isfinite(r)])


# ------------------------------------------------------------------ runners
def check_syr2k(ctx, call, ref_C=None):
    """ref_C: the C the oracle sees (beta = 0 cases pass C's triangle zeroed)."""
    uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc = call
    dC = up(ctx, C)
    ctx.dsyr2k(uplo, trans, n, k, alpha, up(ctx, A), lda, up(ctx, B), ldb, beta, dC, ldc)
    got = dC.to_host()
    Cr = C if ref_C is None else ref_C
    ref, d1, d2 = orc.ssyr2k_ld(uplo, trans, n, k, alpha, A, lda, B, ldb, beta, Cr, ldc)
    idx = region(n, n, ldc, uplo)
    bound = EPS_DD * ((k + 2) * abs(alpha) * d1 + (k + 1) * abs(alpha) * d2 + 2 * c_term(beta, Cr))
    assert ieee_factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F64)[keep])
    return got


def check_symm(ctx, call, ref_C=None):
    side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc = call
    dC = up(ctx, C)
    ctx.dsymm(side, uplo, m, n, alpha, up(ctx, A), lda, up(ctx, B), ldb, beta, dC, ldc)
    got = dC.to_host()
    Cr = C if ref_C is None else ref_C
    ref, ad = orc.ssymm_ld(side, uplo, m, n, alpha, A, lda, B, ldb, beta, Cr, ldc)
    order = m if side == 1 else n
    idx = region(m, n, ldc)
    bound = EPS_DD * ((order + 2) * abs(alpha) * ad + 3 * c_term(beta, Cr))
    assert ieee_factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F64)[keep])
    return got


def check_trmm(ctx, call):
    side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb = call
    dB = up(ctx, B)
    ctx.dtrmm(side, uplo, trans, unit, m, n, alpha, up(ctx, A), lda, dB, ldb)
    got = dB.to_host()
    ref, ad = orc.strmm_ld(*call)
    order = m if side == 1 else n
    idx = region(m, n, ldb)
    assert ieee_factor(got, ref, EPS_DD * (order + 2) * abs(alpha) * ad, idx) <= 1
    keep = outside(len(B), idx)
    assert bits_equal(got[keep], np.asarray(B, F64)[keep])
    return got


# ------------------------------------------------------------ edge cases
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases(ctx, cm):
    # tests/{dsyr2k,dsymm,dtrmm}/edge-cases*.json through the layout mapping
    for c in rc.load("dsyr2k", cm):
        check_syr2k(ctx, rc.syr2k_call(c, F64))
    for c in rc.load("dsymm", cm):
        check_symm(ctx, rc.symm_call(c, F64))
    for c in rc.load("dtrmm", cm):
        check_trmm(ctx, rc.tri_call(c, F64))


# ------------------------------------------------------------ dsyr2k
def syr2k_case(layout, N, K, uplo, trans, alpha=1.5, beta=0.5, seeds=(71, 72, 73)):
    # tests/dsyr2k/src/test.dsyr2k.js:192-265: op(A) N x K, ld = stored columns
    aR, aC = (N, K) if trans == "no-transpose" else (K, N)
    ld = aR if layout == "column-major" else aC
    return dict(layout=layout, uplo=uplo, trans=trans, n=N, k=K, alpha=alpha, beta=beta,
                A=orc.random_f64(aR * aC, -1, 1, seeds[0]), lda=ld,
                B=orc.random_f64(aR * aC, -1, 1, seeds[1]), ldb=ld,
                C=orc.random_f64(N * N, -1, 1, seeds[2]), ldc=N)


@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("N", [150, 400])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
def test_dsyr2k_multi_tile(ctx, layout, N, uplo, trans):
    check_syr2k(ctx, rc.syr2k_call(syr2k_case(layout, N, 9, uplo, trans), F64))


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("n,k", [(4224, 272), (1100, 48)])
def test_dsyr2k_one_launch(ctx, uplo, trans, n, k):
    # lda == ldb and k a multiple of 16: one launch over (A, B) then (B, A).
    # 4224 / 272: 561 tiles of 128, a split-k tail whose k-slices straddle
    # the switch (k-tile 17 of 34); 1100 / 48: 64 tier with edge tiles
    from tests.test_gpu_level3 import syr2k_sampled

    print(f"dsyr2k one launch uplo={uplo} trans={trans} n={n} k={k}", flush=True)
    ld = (k if trans else n) + 2
    syr2k_sampled(ctx, uplo, trans, n, k, 0.75, -0.5, ld, n + 1, 2000 + n, np.float64)


@pytest.mark.parametrize("uplo", [1, 2])
def test_dsyr2k_k0_is_beta_c(ctx, uplo):
    # test.dsyr2k.js:267-319: k = 0 gives beta C on the triangle (exact in
    # fp64), the other triangle unchanged
    n = 4
    C = orc.random_f64(n * n, -5, 5, 310 + uplo)
    dC = up(ctx, C)
    ctx.dsyr2k(uplo, 0, n, 0, 1.5, up(ctx, np.zeros(n)), n, up(ctx, np.zeros(n)), n, 0.5, dC, n)
    got = dC.to_host()
    idx = region(n, n, n, uplo)
    want = C.copy()
    want[idx] = 0.5 * C[idx]
    assert bits_equal(got, want)


def test_dsyr2k_quick_return_and_other_triangle(ctx):
    # test.dsyr2k.js:364-416: alpha = 0 or k = 0 with beta = 1 returns C bit
    # for bit; the unreferenced triangle is never written
    n = 7
    C = orc.random_f64(n * n, -1, 1, 1060) * np.pi
    for alpha, k in ((0.0, 3), (1.5, 0)):
        kk = max(k, 1)
        dC = up(ctx, C)
        ctx.dsyr2k(1, 0, n, k, alpha, up(ctx, orc.random_f64(n * kk, -1, 1, 1) * np.e), n,
                   up(ctx, orc.random_f64(n * kk, -1, 1, 2) * np.e), n, 1.0, dC, n)
        assert bits_equal(dC.to_host(), C)
    for uplo in (1, 2):
        A = orc.random_f64(n * 3, -1, 1, 3) * np.e
        B = orc.random_f64(n * 3, -1, 1, 4) * np.e
        check_syr2k(ctx, (uplo, 0, n, 3, 1.5, A, n, B, n, 0.5, C, n))


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 150])
def test_dsyr2k_ieee_special_values(ctx, uplo, n):
    # test.dsyr2k.js:418-472: Inf in A, NaN in B propagate; beta = 0 ignores
    # NaN / Inf in C's triangle, the other triangle keeps them
    c = dict(layout="row-major", uplo=uplo, trans="no-transpose", n=n, k=n, alpha=1.5, beta=0.0,
             A=orc.random_f64(n * n, -1, 1, 1), lda=n, B=orc.random_f64(n * n, -1, 1, 2), ldb=n,
             C=orc.random_f64(n * n, -1, 1, 3), ldc=n)
    c["A"][at(n, 4, 2)] = np.inf
    c["B"][at(n, 3, 1)] = np.nan
    c["C"][at(n, 2, 2)] = np.nan
    c["C"][at(n, 0, n - 1)] = np.nan
    c["C"][at(n, n - 1, 0)] = np.inf
    call = rc.syr2k_call(c, F64)
    # the oracle sees C's triangle zeroed (beta = 0 ignores it)
    Cz = call[10].copy()
    Cz[region(n, n, n, call[0])] = 0.0
    got = check_syr2k(ctx, call, ref_C=Cz)
    assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 150])
def test_dsyr2k_f64_exponent_range(ctx, uplo, n):
    # the inputs of test.dsyr2k.js:474-554, in f64's range: 1e300 and 1e-50
    # are read as they are and a result past 3.4e38 stays finite
    c = dict(layout="row-major", uplo=uplo, trans="no-transpose", n=n, k=n, alpha=1.5, beta=0.5,
             A=orc.random_f64(n * n, -1, 1, 1), lda=n, B=orc.random_f64(n * n, -1, 1, 2), ldb=n,
             C=orc.random_f64(n * n, -1, 1, 3), ldc=n)
    c["A"][at(n, 4, 2)], c["A"][at(n, 5, 5)] = 1e300, 1e-50
    c["C"][at(n, 0, n - 1)], c["C"][at(n, n - 1, 0)] = 1e300, -1e300
    got = check_syr2k(ctx, rc.syr2k_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    c = dict(c, alpha=10.0, A=orc.random_f64(n * n, -1, 1, 1), C=orc.random_f64(n * n, -1, 1, 3))
    c["A"][at(n, 3, 3)] = 3e38
    got = check_syr2k(ctx, rc.syr2k_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e39


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 150])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_dsyr2k_alpha0_reads_neither_a_nor_b(ctx, uplo, n, beta):
    # test.dsyr2k.js:559-603
    c = syr2k_case("row-major", n, n, uplo, "no-transpose", alpha=0.0, beta=beta, seeds=(1, 2, 3))
    c["A"][at(n, 1, 2)], c["A"][at(n, 3, 0)], c["B"][at(n, 2, 3)] = np.nan, -np.inf, np.inf
    if beta == 0:
        c["C"][at(n, 4, 4)] = np.nan
    call = rc.syr2k_call(c, F64)
    Cr = call[10].copy()
    if beta == 0:
        Cr[region(n, n, n, call[0])] = 0.0
    got = check_syr2k(ctx, call, ref_C=Cr)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_dsyr2k_large_tier_padded(ctx, uplo, trans):
    n, k = 1100, 333
    lda = (k if trans else n) + 3
    ldb = (k if trans else n) + 1
    ldc = n + 2
    cols = n if trans else k
    call = (uplo, trans, n, k, 0.75, orc.random_f64(lda * cols, -1, 1, 5), lda,
            orc.random_f64(ldb * cols, -1, 1, 6), ldb, -1.25, orc.random_f64(ldc * n, -1, 1, 7), ldc)
    check_syr2k(ctx, call)


def _cm_transpose(X, rows, cols, ld):
    """Column-major rows x cols (leading dimension ld) -> its transpose as a
    dense column-major cols x rows array (leading dimension cols)."""
    M = np.asarray(X, F64)[: ld * cols].reshape(cols, ld)[:, :rows]
    return np.ascontiguousarray(M.T).reshape(-1)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_dsyr2k_operands_of_different_storage_orders(ctx, uplo, ta, tb):
    # GpuMatrix A and B of different layouts (src/dsyr2k/dsyr2k.mjs:87-90, 150-151)
    # reach one wgb_dsyr2k call with a flag per operand
    n, k = 333, 150
    lda = (k if ta else n) + 2
    ldb = (k if tb else n) + 1
    ldc = n + 4
    A = orc.random_f64(lda * (n if ta else k), -1, 1, 64)
    B = orc.random_f64(ldb * (n if tb else k), -1, 1, 65)
    C = orc.random_f64(ldc * n, -1, 1, 66)
    dC = up(ctx, C)
    ctx.dsyr2k(uplo, ta, n, k, 0.75, up(ctx, A), lda, up(ctx, B), ldb, -0.5, dC, ldc, transB=tb)
    got = dC.to_host()
    rows_b, cols_b = (k, n) if tb else (n, k)
    Bc = _cm_transpose(B, rows_b, cols_b, ldb)
    ref, d1, d2 = orc.ssyr2k_ld(uplo, ta, n, k, 0.75, A, lda, Bc, cols_b, -0.5, C, ldc)
    idx = region(n, n, ldc, uplo)
    bound = EPS_DD * ((k + 2) * 0.75 * d1 + (k + 1) * 0.75 * d2 + 2 * c_term(-0.5, C))
    assert factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], C[keep])


# ------------------------------------------------------------ dsymm
def symm_case(layout, side, uplo, N, OTHER, pad, alpha=1.5, beta=0.5, seeds=(91, 92, 93)):
    # tests/dsymm/src/test.dsymm.js:174-220
    m = N if side == "left" else OTHER
    n = OTHER if side == "left" else N
    cm = layout == "column-major"
    LD = (m if cm else n) + pad
    OUTER = n if cm else m
    return dict(layout=layout, side=side, uplo=uplo, m=m, n=n, alpha=alpha, beta=beta,
                A=orc.random_f64(N * N, -1, 1, seeds[0]), lda=N,
                B=orc.random_f64(OUTER * LD, -1, 1, seeds[1]), ldb=LD,
                C=orc.random_f64(OUTER * LD, -1, 1, seeds[2]), ldc=LD)


@pytest.mark.parametrize("N,pad", [(150, 1), (400, 4)])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_dsymm_multi_tile(ctx, N, pad, layout, side, uplo):
    check_symm(ctx, rc.symm_call(symm_case(layout, side, uplo, N, 72, pad), F64))


@pytest.mark.parametrize("mn", [(0, 4), (4, 0)])
def test_dsymm_zero_dimension(ctx, mn):
    # test.dsymm.js:143-172: C comes back as it was
    m, n = mn
    C = orc.random_f64(16, -5, 5, 300 + m)
    dC = up(ctx, C)
    # the C ABI checks lda / ldb before the quick return, as reference BLAS
    ctx.dsymm(1, 1, m, n, 1.5, up(ctx, np.zeros(0)), max(1, m), up(ctx, np.zeros(0)), max(1, m), 0.5,
              dC, 4)
    assert bits_equal(dC.to_host(), C)


def test_dsymm_quick_return_and_ldc_padding(ctx):
    # test.dsymm.js:249-295: alpha = 0 with beta = 1 returns C bit for bit;
    # C's ld padding is never written
    n = 6
    full = lambda size, s: orc.random_f64(size, -1, 1, s) * np.pi  # noqa: E731
    C = full(n * n, 1070)
    dC = up(ctx, C)
    ctx.dsymm(1, 1, n, n, 0.0, up(ctx, full(n * n, 1)), n, up(ctx, full(n * n, 2)), n, 1.0, dC, n)
    assert bits_equal(dC.to_host(), C)
    for side in (1, 2):
        m, ldc = 4, n + 3
        order = m if side == 1 else n
        check_symm(ctx, (side, 2, m, n, 1.5, full(order * order, 3), order, full(m * n, 4), m, 0.5,
                         full(ldc * n, 5), ldc))


@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 150])
def test_dsymm_ieee_special_values(ctx, side, uplo, n):
    # test.dsymm.js:297-327: Inf in A's stored triangle and NaN in B
    # propagate; beta = 0 ignores NaN / Inf in C
    stored = (4, 2) if uplo == "lower" else (2, 4)
    c = symm_case("row-major", side, uplo, n, n, 0, beta=0.0, seeds=(1, 2, 3))
    c["A"][at(n, *stored)] = np.inf
    c["B"][at(n, 3, 1)] = np.nan
    c["C"][at(n, 2, 2)], c["C"][at(n, n - 1, 0)] = np.nan, np.inf
    call = rc.symm_call(c, F64)
    got = check_symm(ctx, call, ref_C=np.zeros_like(call[10]))
    assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_dsymm_unstored_triangle_not_read(ctx, uplo):
    # test.dsymm.js:328-355
    n = 7
    unstored = (1, 5) if uplo == "lower" else (5, 1)
    c = symm_case("row-major", "left", uplo, n, n, 0, seeds=(4, 5, 6))
    c["A"][at(n, *unstored)] = np.nan
    assert np.all(np.isfinite(check_symm(ctx, rc.symm_call(c, F64))))


@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("n", [7, 150])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_dsymm_alpha0_reads_neither_a_nor_b(ctx, side, n, beta):
    # test.dsymm.js:409-438
    c = symm_case("row-major", side, "lower", n, n, 0, alpha=0.0, beta=beta, seeds=(1, 2, 3))
    c["A"][at(n, 3, 1)], c["B"][at(n, 2, 3)] = np.nan, np.inf
    if beta == 0:
        c["C"][at(n, 4, 4)] = np.nan
    call = rc.symm_call(c, F64)
    ref_C = np.zeros_like(call[10]) if beta == 0 else None
    assert np.all(np.isfinite(check_symm(ctx, call, ref_C=ref_C)))


@pytest.mark.parametrize("side", [1, 2])
@pytest.mark.parametrize("uplo", [1, 2])
def test_dsymm_large_and_b_other_storage_order(ctx, side, uplo):
    m, n = (1500, 700) if side == 1 else (700, 1500)
    order = m if side == 1 else n
    lda, ldb, ldc = order + 1, m + 4, m + 3
    call = (side, uplo, m, n, 1.0, orc.random_f64(lda * order, -1, 1, 8), lda,
            orc.random_f64(ldb * n, -1, 1, 9), ldb, 0.25, orc.random_f64(ldc * n, -1, 1, 10), ldc)
    check_symm(ctx, call)
    # B stored in the other order (src/dsymm/dsymm.mjs:87-90, 156-165): op(B) = B^T
    ldb_t = n + 3
    Bt = orc.random_f64(ldb_t * m, -1, 1, 62)
    A, C = call[5], call[10]
    dC = up(ctx, C)
    ctx.dsymm(side, uplo, m, n, 1.25, up(ctx, A), lda, up(ctx, Bt), ldb_t, 0.5, dC, ldc, transB=1)
    got = dC.to_host()
    ref, ad = orc.ssymm_ld(side, uplo, m, n, 1.25, A, lda, _cm_transpose(Bt, n, m, ldb_t), m, 0.5,
                           C, ldc)
    idx = region(m, n, ldc)
    bound = EPS_DD * ((order + 2) * 1.25 * ad + 3 * c_term(0.5, C))
    assert factor(got, ref, bound, idx) <= 1
    assert bits_equal(got[outside(len(C), idx)], C[outside(len(C), idx)])


# ------------------------------------------------------------ dtrmm
def tri_case(layout, side, uplo, transA, diag, N, OTHER, pad, alpha=1.5, seeds=(81, 82)):
    # tests/dtrmm/src/test.dtrmm.js:173-222
    m = N if side == "left" else OTHER
    n = OTHER if side == "left" else N
    cm = layout == "column-major"
    LD = (m if cm else n) + pad
    OUTER = n if cm else m
    return dict(layout=layout, side=side, uplo=uplo, transA=transA, diag=diag, m=m, n=n,
                alpha=alpha, A=orc.random_f64(N * N, -1, 1, seeds[0]), lda=N,
                B=orc.random_f64(OUTER * LD, -1, 1, seeds[1]), ldb=LD)


COMBOS = list(itertools.product(["row-major", "column-major"], ["left", "right"], ["lower", "upper"],
                                ["no-transpose", "transpose"]))


@pytest.mark.parametrize("N,pad", [(150, 1), (400, 4)])
@pytest.mark.parametrize("layout,side,uplo,transA", COMBOS)
def test_dtrmm_multi_tile(ctx, N, pad, layout, side, uplo, transA):
    diag = "unit" if transA == "transpose" else "non-unit"
    check_trmm(ctx, rc.tri_call(tri_case(layout, side, uplo, transA, diag, N, 72, pad), F64))


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
@pytest.mark.parametrize("unit", [0, 1])
@pytest.mark.parametrize("dims", [(3000, 2900), (700, 260)])
def test_dtrmm_large_unreferenced_nan(ctx, side, uplo, trans, unit, dims):
    # 128-tiles with edge tiles, and 64-tiles; NaN wherever A is not
    # referenced
    from tests.test_gpu_level3 import trmm_sampled

    m, n = dims
    order = m if side == 1 else n
    print(f"dtrmm side={side} uplo={uplo} trans={trans} unit={unit} {m}x{n}", flush=True)
    trmm_sampled(ctx, side, uplo, trans, unit, m, n, 0.75, order + 2, m + 3, 88 + order, np.float64)


@pytest.mark.parametrize("mn", [(0, 4), (4, 0)])
def test_dtrmm_zero_dimension(ctx, mn):
    # test.dtrmm.js:141-171
    m, n = mn
    B = orc.random_f64(16, -5, 5, 400 + m)
    dB = up(ctx, B)
    ctx.dtrmm(1, 1, 0, 0, m, n, 1.5, up(ctx, np.zeros(0)), max(1, m), dB, 4)
    assert bits_equal(dB.to_host(), B)


@pytest.mark.parametrize("side", [1, 2])
def test_dtrmm_ldb_padding(ctx, side):
    # test.dtrmm.js:252-281
    m, n = 4, 6
    ldb = m + 3
    order = m if side == 1 else n
    check_trmm(ctx, (side, 2, 0, 0, m, n, 1.5, orc.random_f64(order * order, -1, 1, 1) * np.pi,
                     order, orc.random_f64(ldb * n, -1, 1, 2) * np.pi, ldb))


@pytest.mark.parametrize("data,ldb", [([1, 2, 99, 3, 4], 3), ([1, 2, 3, 4, 7, 8], 2)])
def test_dtrmm_b_storage_length(ctx, data, ldb):
    # test.dtrmm.js:283-311: B holds exactly the elements its layout names
    # (row-major 2 x 2, lower A = [[2, 0], [3, 4]]); small integers, so exact
    c = dict(layout="row-major", side="left", uplo="lower", transA="no-transpose", diag="non-unit",
             m=2, n=2, alpha=1.0, A=[2, 0, 3, 4], lda=2, B=data, ldb=ldb)
    call = rc.tri_call(c, F64)
    got = check_trmm(ctx, call)
    assert len(got) == len(data)
    ref, _ = orc.strmm_ld(*call)
    assert np.array_equal(got, ref)
    # the row-major product [[2, 0], [3, 4]] @ [[1, 2], [3, 4]]
    Bm = got
    want = np.array([[2.0, 4.0], [15.0, 22.0]])
    assert np.array_equal(np.array([[Bm[0], Bm[1]], [Bm[ldb], Bm[ldb + 1]]]), want)


@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("transA", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 150])
def test_dtrmm_ieee_special_values(ctx, side, uplo, transA, n):
    # test.dtrmm.js:313-343: Inf and NaN in A's stored triangle propagate
    stored = (4, 2) if uplo == "lower" else (2, 4)
    stored_nan = (6, 1) if uplo == "lower" else (1, 6)
    c = tri_case("row-major", side, uplo, transA, "non-unit", n, n, 0, seeds=(1, 2))
    c["A"][at(n, *stored)] = np.inf
    c["A"][at(n, *stored_nan)] = np.nan
    got = check_trmm(ctx, rc.tri_call(c, F64))
    assert np.isnan(got).any()


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("transA", ["no-transpose", "transpose"])
def test_dtrmm_unstored_triangle_and_unit_diagonal_not_read(ctx, uplo, transA):
    # test.dtrmm.js:344-376
    n = 7
    unstored = (1, 5) if uplo == "lower" else (5, 1)
    c = tri_case("row-major", "left", uplo, transA, "unit", n, n, 0, seeds=(4, 5))
    c["A"][at(n, *unstored)] = np.nan
    c["A"][at(n, 3, 3)] = np.nan
    assert np.all(np.isfinite(check_trmm(ctx, rc.tri_call(c, F64))))


@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("n", [7, 150])
def test_dtrmm_f64_exponent_range(ctx, side, n):
    # the inputs of test.dtrmm.js:378-423 in f64's range
    c = tri_case("row-major", side, "lower", "no-transpose", "non-unit", n, n, 0, seeds=(1, 2))
    c["A"][at(n, 4, 2)], c["A"][at(n, 5, 5)] = 1e300, 1e-50
    got = check_trmm(ctx, rc.tri_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    c = tri_case("row-major", side, "lower", "no-transpose", "non-unit", n, n, 0, alpha=10.0,
                 seeds=(1, 2))
    c["A"][at(n, 3, 3)] = 3e38
    got = check_trmm(ctx, rc.tri_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e39


@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("n", [7, 150])
def test_dtrmm_alpha0_reads_neither_a_nor_b(ctx, side, n):
    # test.dtrmm.js:427-452: B becomes zero, NaN / Inf in A and B never read
    c = tri_case("row-major", side, "lower", "no-transpose", "non-unit", n, n, 0, alpha=0.0,
                 seeds=(1, 2))
    c["A"][at(n, 3, 1)], c["B"][at(n, 2, 3)], c["B"][0] = np.nan, np.inf, np.nan
    side_, uplo_, trans, unit, m, n_, alpha, A, lda, B, ldb = rc.tri_call(c, F64)
    dB = up(ctx, B)
    ctx.dtrmm(side_, uplo_, trans, unit, m, n_, alpha, up(ctx, A), lda, dB, ldb)
    got = dB.to_host()
    assert bits_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
def test_dtrmm_large(ctx, side, uplo, trans):
    m, n = (1500, 900) if side == 1 else (900, 1500)
    order = m if side == 1 else n
    lda, ldb = order + 2, m + 1
    call = (side, uplo, trans, 0, m, n, 0.5, orc.random_f64(lda * order, -1, 1, 11), lda,
            orc.random_f64(ldb * n, -1, 1, 12), ldb)
    check_trmm(ctx, call)
