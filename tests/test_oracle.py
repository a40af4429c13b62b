"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked against something independent of its own
code: the reference's golden vectors (random_golden.json, written by the
reference module itself), hand-derived values of the reference's edge-case
fixtures, numpy library routines on exact (integer-valued) inputs, closed
forms, brute force, and mathematical invariants. A few tests plant a mistake
in an oracle result and check that the parity metric rejects it.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import orc
from tests import refcases
from tests.helpers import EPS32, gemm_forward_factor, ulp_diff32

GOLDEN = refcases.GOLDEN


# ---------------------------------------------------------------- mulberry32
def test_random_matches_reference_golden():
    with open(os.path.join(GOLDEN, "random_golden.json")) as f:
        gold = json.load(f)
    assert gold["source"] == "src/random/random.mjs"
    for case in gold["cases"]:
        idx = np.array(case["index"])
        f32 = orc.random_f32(case["n"], case["low"], case["high"], case["seed"])
        f64 = orc.random_f64(case["n"], case["low"], case["high"], case["seed"])
        assert np.array_equal(f32.view(np.uint32)[idx], np.array(case["f32_bits"], np.uint32)), case
        assert np.array_equal(f64[idx], np.array(case["f64"], np.float64)), case


def test_random_is_a_mulberry_stream():
    # draw i of a stream is a function of seed + (i+1)*step alone: the f64
    # stream of low=0, high=1 is the raw unit draws, and f32(-1,1) is
    # -1 + 2u rounded (an exact double), so the two must agree everywhere.
    u = orc.random_f64(4096, 0.0, 1.0, 77)
    assert np.all((u >= 0) & (u < 1))
    f = orc.random_f32(4096, -1.0, 1.0, 77)
    assert np.array_equal(f, (-1.0 + 2.0 * u).astype(np.float32))


def test_normal_sampler_invariants():
    # Box-Muller over the unit draws: z0^2 + z1^2 = -2 ln(1-u1), atan2(z1, z0) = 2 pi u2.
    n = 20000
    z = orc.random_normal_f32(n, 5).astype(np.float64)
    u = orc.random_f64(n, 0.0, 1.0, 5)
    u1, u2 = u[0::2], u[1::2]
    r2 = z[0::2] ** 2 + z[1::2] ** 2
    want = -2.0 * np.log1p(-u1)
    assert np.allclose(r2, want, rtol=1e-6, atol=1e-12)
    ang = np.mod(np.arctan2(z[1::2], z[0::2]), 2 * np.pi)
    d = np.abs(ang - 2 * np.pi * u2)
    d = np.minimum(d, 2 * np.pi - d)
    big = r2 > 1e-6
    assert np.max(d[big]) < 1e-5
    big_sample = orc.random_normal_f32(1 << 20, 1).astype(np.float64)
    assert abs(big_sample.mean()) < 5e-3 and abs(big_sample.std() - 1) < 5e-3


def test_normal_sampler_odd_length_is_prefix():
    a = orc.random_normal_f32(1001, 9)
    b = orc.random_normal_f32(1002, 9)
    assert np.array_equal(a, b[:1001])


# ------------------------------------------------------------ level 1 fixtures
# Hand-derived results of the reference's edge cases (tests/<routine>/edge-cases.json).
SDOT_EXPECT = [0.0, 25.0, 0.0, 0.0, 11.0, 12.0]
SASUM_EXPECT = [9.0, 205.0, 0.0, 7.0, 6.0]
ISAMAX_EXPECT = [0, 0, 1, 1, 0, 3, 0, 1, 0, 1, 1]


def test_sdot_edge_cases():
    for case, want in zip(refcases.load("sdot"), SDOT_EXPECT):
        x = np.array(case["x"], np.float32)
        y = np.array(case["y"], np.float32)
        got = orc.sdot_wgsl(case["n"], x, case["incx"], y, case["incy"])
        assert got == np.float32(want), case["label"]
        s, _ = orc.dot_ld(case["n"], x, case["incx"], y, case["incy"])
        assert s == want, case["label"]


def test_sasum_edge_cases():
    for case, want in zip(refcases.load("sasum"), SASUM_EXPECT):
        x = np.array(case["x"], np.float32)
        assert orc.sasum_wgsl(case["n"], x, case["incx"]) == np.float32(want), case["label"]
        assert orc.sum_abs_ld(case["n"], x, case["incx"]) == want


def test_snrm2_edge_cases():
    f = np.float32
    expect = [f(5), f(5), f(1), f(0), f(5), f(5), f(3e19), f(3e19), None]
    for case, want in zip(refcases.load("snrm2"), expect):
        x = np.array(case["x"], np.float32)
        got = orc.snrm2_wgsl(case["n"], x, case["incx"])
        assert np.isfinite(got), case["label"]
        if want is None:  # [1e-20]*3: sqrt(3)*fround(1e-20), within 1 ULP (parity unpinned at the bit)
            want = f(math.sqrt(3.0) * float(f(1e-20)))
            assert ulp_diff32(got, want) <= 1, (got, want)
        else:
            assert got == want, (case["label"], got, want)


def test_isamax_edge_cases_and_nan_rules():
    for case, want in zip(refcases.load("isamax"), ISAMAX_EXPECT):
        x = np.array(case["x"], np.float32)
        assert orc.isamax_wgsl(case["n"], x, case["incx"]) == want, case["label"]
        assert orc.isamax_brute(case["n"], x, case["incx"]) == want, case["label"]
    N, I = np.nan, np.inf
    # tests/isamax/src/test.isamax.js:97-139
    for arr, want in [([1, N, 7, 3], 2), ([1, 2, 3, N], 2), ([N, N, N, N], 0), ([N, 5, 2, 3], 1),
                      ([N, I, 2, 3], 1), ([1, I, 2, 3], 1), ([1, -I, 2, 3], 1)]:
        x = np.array(arr, np.float32)
        assert orc.isamax_wgsl(len(x), x, 1) == want, arr
        assert orc.isamax_brute(len(x), x, 1) == want, arr
    for n in (0, -3):
        assert orc.isamax_wgsl(n, np.ones(2, np.float32), 1) == -1
        assert orc.isamax_brute(n, np.ones(2, np.float32), 1) == -1


def test_level1_zero_length():
    x = orc.random_f32(8, -1, 1, 300)
    assert orc.sdot_wgsl(0, x, 1, x, 1) == 0
    assert orc.sasum_wgsl(0, x, 1) == 0
    assert orc.snrm2_wgsl(0, x, 1) == 0


# ------------------------------------------------- level 1 vs extended sums
@pytest.mark.parametrize("n,inc", [(1, 1), (7, 1), (8192 * 4 - 1, 1), (8192 * 4 + 5, 1),
                                   (100003, 1), (30001, 3)])
def test_wgsl_reductions_within_reference_bounds(n, inc):
    x = orc.random_f32((n - 1) * inc + 1, -1, 1, 11)
    y = orc.random_f32((n - 1) * inc + 1, -1, 1, 12)
    s, a = orc.dot_ld(n, x, inc, y, inc)
    # numpy float64 dot on the strided views agrees with the long-double sum
    xs, ys = x[::inc][:n].astype(np.float64), y[::inc][:n].astype(np.float64)
    assert abs(np.dot(xs, ys) - s) <= 1e-12 * a
    assert abs(float(orc.sdot_wgsl(n, x, inc, y, inc)) - s) <= n * EPS32 * a
    asum = orc.sum_abs_ld(n, x, inc)
    assert asum == pytest.approx(np.sum(np.abs(xs)), rel=1e-13)
    assert ulp_diff32(orc.sasum_wgsl(n, x, inc), np.float32(asum)) <= 50
    nrm = orc.nrm2_ld(n, x, inc)
    assert nrm == pytest.approx(np.linalg.norm(xs), rel=1e-13)
    assert ulp_diff32(orc.snrm2_wgsl(n, x, inc), np.float32(nrm)) <= 50
    assert orc.isamax_wgsl(n, x, inc) == orc.isamax_brute(n, x, inc) == int(np.argmax(np.abs(xs)))


SNRM2_REGIMES = [
    ("medium only", lambda i: np.sin(i) * 3),
    ("big + medium", lambda i: np.where(i % 4096 == 7, 1e30, np.cos(i))),
    ("near f32 max", lambda i: np.where(i % 65536 == 3, 1e37, 1.0)),
    ("small + medium", lambda i: np.where(i % 1024 == 0, 1e-5, 1e-25 * (1 + (i % 7)))),
    ("small only", lambda i: 1e-30 * (1 + (i % 5))),
    ("straddling", lambda i: np.array([2.0 ** 50 * 1.5, 2.0 ** 50 * 0.75, 2.0 ** -63 * 1.5,
                                       2.0 ** -63 * 0.75, 1.0])[i % 5]),
]


@pytest.mark.parametrize("label,gen", SNRM2_REGIMES, ids=[r[0] for r in SNRM2_REGIMES])
@pytest.mark.parametrize("inc", [1, 3])
def test_snrm2_wgsl_magnitude_regimes(label, gen, inc):
    # tests/snrm2/src/test.snrm2.js:92-130 at n = 2^20
    N = 1 << 20
    x = np.zeros((N - 1) * inc + 1, np.float32)
    x[::inc] = gen(np.arange(N)).astype(np.float32)
    want = np.float32(np.sqrt(np.sum(x[::inc].astype(np.float64) ** 2)))
    got = orc.snrm2_wgsl(N, x, inc)
    assert np.isfinite(got)
    assert ulp_diff32(got, want) <= 50, (got, want)


def test_snrm2_wgsl_specials():
    N = 1 << 16
    x = orc.random_f32(N, -1, 1, 7)
    x[12345] = np.inf
    assert orc.snrm2_wgsl(N, x, 1) == np.inf
    x = orc.random_f32(N, -1, 1, 8)
    x[54321] = np.nan
    assert np.isnan(orc.snrm2_wgsl(N, x, 1))
    x = orc.random_f32(N, -1, 1, 9)
    x[1], x[2], x[999] = 1e30, 1e-30, np.nan
    assert np.isnan(orc.snrm2_wgsl(N, x, 1))


def test_nrm_combine_closed_forms():
    # medium only: sqrt(amed); big only: 2^76*sqrt(abig); small only: 2^-75*sqrt(asml)
    assert orc.nrm_combine(0.0, 25.0, 0.0) == 5.0
    assert orc.nrm_combine(4.0, 0.0, 0.0) == np.float32(2.0 ** 77)
    assert orc.nrm_combine(0.0, 0.0, 1024.0) == np.float32(2.0 ** -70)
    assert np.isnan(orc.nrm_combine(1.0, np.nan, 1.0))
    # big + medium: medium folds in at big's scale (2^-152)
    assert orc.nrm_combine(1.0, 2.0 ** 100, 0.0) == np.float32(2.0 ** 76 * math.sqrt(1.0 + 2.0 ** -52))
    # small + medium: |x| = {2^-60 (medium), 2^-64 (small)} -> sqrt(2^-120 + 2^-128)
    got = orc.nrm_combine(0.0, 2.0 ** -120, (2.0 ** -64 * 2.0 ** 75) ** 2)
    assert ulp_diff32(got, np.float32(math.sqrt(2.0 ** -120 + 2.0 ** -128))) <= 1


def test_planted_reduction_mistakes_are_caught():
    # a dropped (large) term, a wrong stride and a wrong tie rule must fail
    # the reference's own metrics
    n = 5000
    x = orc.random_f32(n, -1, 1, 21)
    y = orc.random_f32(n, -1, 1, 22)
    x[n - 1] = 1000.0
    s, a = orc.dot_ld(n, x, 1, y, 1)
    dropped = float(orc.sdot_wgsl(n - 1, x, 1, y, 1))
    assert abs(dropped - s) > n * EPS32 * a
    half = orc.sasum_wgsl(n // 2, x, 2)
    assert ulp_diff32(half, np.float32(orc.sum_abs_ld(n, x, 1))) > 50
    t = np.array([1, 5, 2, 5, 3], np.float32)
    assert int(np.flatnonzero(np.abs(t) == np.abs(t).max())[-1]) != orc.isamax_wgsl(5, t, 1)


# --------------------------------------------------------------------- GEMM
SGEMM_EXPECT_ROW_MAJOR = [
    [2, 4, 6, 8], [5, 6, 7, 8], [4, 5, 10, 11], [4, 5, 10, 11], [4, 5, 10, 11], [4, 5, 10, 11],
    [4, 5, 10, 11], [4, 5, 10, 11], [4, 5, 99, 10, 11, 99], [10, 12, 15, 18, 20, 24],
]


def test_sgemm_edge_cases_hand_values():
    for case, want in zip(refcases.load("sgemm"), SGEMM_EXPECT_ROW_MAJOR):
        call = refcases.gemm_call(case, np.float64)
        out, _ = orc.gemm_ld(*call)
        assert np.array_equal(out, np.array(want, np.float64)), case["label"]
        out32 = orc.sgemm_wgsl(*call)
        assert np.array_equal(out32, np.array(want, np.float32)), case["label"]


@pytest.mark.parametrize("routine", ["sgemm", "dgemm", "sgemmtr", "dgemmtr"])
@pytest.mark.parametrize("cm", [False, True])
def test_gemm_edge_cases_match_numpy(routine, cm):
    for case in refcases.load(routine, cm):
        call = refcases.gemm_call(case, np.float64)
        want = refcases.numpy_gemm(*call)
        out, _ = orc.gemm_ld(*call)
        assert np.array_equal(out, want), case["label"]
        if not routine.startswith("d"):
            assert np.array_equal(orc.sgemm_wgsl(*call), want.astype(np.float32)), case["label"]


@pytest.mark.parametrize("routine", ["ssyrk", "dsyrk"])
@pytest.mark.parametrize("cm", [False, True])
def test_syrk_edge_cases_match_numpy(routine, cm):
    for case in refcases.load(routine, cm):
        uplo, trans, n, k, alpha, A, lda, beta, C, ldc = refcases.syrk_call(case, np.float64)
        call = (uplo, trans, 1 - trans, n, n, k, alpha, A, lda, A, lda, beta, C, ldc)
        want = refcases.numpy_gemm(*call)
        out, _ = orc.gemm_ld(*call)
        assert np.array_equal(out, want), case["label"]


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("uplo", [0, 1, 2])
def test_gemm_ld_random_vs_numpy_and_wgsl_bound(ta, tb, uplo):
    m, n, k = 37, 29, 45
    lda = (k if ta else m) + 3
    ldb = (n if tb else k) + 1
    ldc = m + 2
    A = orc.random_f32(lda * (m if ta else k), -1, 1, 1).astype(np.float64)
    B = orc.random_f32(ldb * (k if tb else n), -1, 1, 2).astype(np.float64)
    C = orc.random_f32(ldc * n, -1, 1, 3).astype(np.float64)
    alpha, beta = 1.5, 0.5
    out, absdot = orc.gemm_ld(uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    want = refcases.numpy_gemm(uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    assert np.allclose(out, want, rtol=1e-13, atol=1e-13)
    w32 = orc.sgemm_wgsl(uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    assert gemm_forward_factor(w32, out, absdot, C, m, n, k, alpha, beta, ldc, uplo) <= 1.0
    # planted mistakes: transposed operand, dropped beta term, one k term short
    bad_t, _ = orc.gemm_ld(uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, -beta, C, ldc)
    assert gemm_forward_factor(bad_t, out, absdot, C, m, n, k, alpha, beta, ldc, uplo) > 1.0
    bad_k, _ = orc.gemm_ld(uplo, ta, tb, m, n, k - 1, alpha, A, lda, B, ldb, beta, C, ldc)
    assert gemm_forward_factor(bad_k, out, absdot, C, m, n, k, alpha, beta, ldc, uplo) > 1.0


def test_gemm_alpha_zero_and_beta_zero_rules():
    n = 7
    A = orc.random_f32(n * n, -1, 1, 1).astype(np.float64)
    B = orc.random_f32(n * n, -1, 1, 2).astype(np.float64)
    C = orc.random_f32(n * n, -1, 1, 3).astype(np.float64)
    A[1 + 2 * n] = np.nan
    B[2 + 3 * n] = np.inf
    out, _ = orc.gemm_ld(0, 0, 0, n, n, n, 0.0, A, n, B, n, 0.5, C, n)
    assert np.array_equal(out, 0.5 * C)
    C[4 + 4 * n] = np.nan
    out, _ = orc.gemm_ld(0, 0, 0, n, n, n, 0.0, A, n, B, n, 0.0, C, n)
    assert np.array_equal(out, np.zeros_like(C))
    out32 = orc.sgemm_wgsl(0, 0, 0, n, n, n, 0.0, A, n, B, n, 0.0, C, n)
    assert np.array_equal(out32, np.zeros(n * n, np.float32))


def test_sgemm_k0_is_beta_c_bit_exact():
    # tests/sgemm/src/test.sgemm.js:304-351
    C = orc.random_f32(16, -5, 5, 300)
    out32 = orc.sgemm_wgsl(0, 0, 1, 4, 4, 0, 1.5, np.zeros(3), 4, np.zeros(3), 4, 0.5, C, 4)
    assert np.array_equal(out32, (np.float32(0.5) * C).astype(np.float32))


# ---- fp64 level 1 (ddot / dasum / dnrm2 / idamax) --------------------------
from fractions import Fraction  # noqa: E402


def _exact(values):
    return sum((Fraction(v) for v in values), Fraction(0))


def _ulps64(a, b):
    if a == b:
        return 0
    ia = np.array(a, np.float64).view(np.int64)
    ib = np.array(b, np.float64).view(np.int64)
    return abs(int(ia) - int(ib))


def test_ddot_dasum_edge_cases_against_exact_rationals():
    # Fixtures: wgblas tests/{ddot,dasum}/edge-cases.json, against the exact
    # rational result of the double inputs: the long-double sums must be
    # within their own precision (n 2^-63 sum|x y|, plus the final rounding).
    for c in refcases.load("ddot"):
        x, y = np.array(c["x"], np.float64), np.array(c["y"], np.float64)
        terms = [Fraction(float(x[i * c["incx"]])) * Fraction(float(y[i * c["incy"]])) for i in range(c["n"])]
        exact = sum(terms, Fraction(0))
        got, sum_abs = orc.ddot_ld(c["n"], x, c["incx"], y, c["incy"])
        tol = c["n"] * 2.0 ** -63 * sum_abs + 2.0 ** -53 * abs(float(exact))
        assert abs(Fraction(got) - exact) <= Fraction(tol), c["label"]
    for c in refcases.load("dasum"):
        x = np.array(c["x"], np.float64)
        want = float(_exact(abs(float(x[i * c["incx"]])) for i in range(c["n"])))
        assert _ulps64(orc.dasum_ld(c["n"], x, c["incx"]), want) <= 1, c["label"]


DNRM2_EXPECT = [5.0, 5.0, 1.0, 0.0, 5.0, 5.0, 3e19, None, math.sqrt(3.0) * 1e-20, None]
IDAMAX_EXPECT = [0, 0, 1, 1, 0, 3, 0, 1, 0, 1, 1, 1]


def test_dnrm2_idamax_edge_cases_hand_values():
    for c, want in zip(refcases.load("dnrm2"), DNRM2_EXPECT):
        x = np.array(c["x"], np.float64)
        got = orc.dnrm2_ld(c["n"], x, c["incx"])
        if want is None:  # sqrt of the exact sum of squares
            want = math.sqrt(float(_exact(Fraction(float(x[i * c["incx"]])) ** 2 for i in range(c["n"]))))
        assert _ulps64(got, want) <= 1, c["label"]
    for c, want in zip(refcases.load("idamax"), IDAMAX_EXPECT):
        assert orc.idamax_brute(c["n"], np.array(c["x"], np.float64), c["incx"]) == want, c["label"]


def test_idamax_nan_rules_and_fp64_specials():
    # tests/idamax/src/test.idamax.js:97-144
    run = lambda a: orc.idamax_brute(len(a), np.array(a, np.float64), 1)
    N, I = np.nan, np.inf
    assert run([1, N, 7, 3]) == 2 and run([1, 2, 3, N]) == 2
    assert run([N, N, N, N]) == 0
    assert run([N, 5, 2, 3]) == 1 and run([N, I, 2, 3]) == 1
    assert run([1, I, 2, 3]) == 1 and run([1, -I, 2, 3]) == 1
    assert orc.idamax_brute(0, np.zeros(1), 1) == -1
    # native f64 range: 1e300 < 1e301 (the reference's double-double reads both as Inf)
    assert run([1e300, 1e301, 5]) == 1
    assert math.isinf(orc.dnrm2_ld(3, np.array([1.0, I, 2.0]), 1))
    assert math.isnan(orc.dnrm2_ld(3, np.array([1.0, I, N]), 1))
    assert orc.dnrm2_ld(2, np.array([3e300, 4e300]), 1) == 5e300


def test_fp64_oracles_agree_with_numpy_on_random_vectors():
    rng = np.random.default_rng(11)
    for n, inc in ((1, 1), (50, 1), (1000, 3), (4097, 2)):
        x = rng.standard_normal((n - 1) * inc + 1)
        y = rng.standard_normal((n - 1) * inc + 1)
        xs, ys = x[::inc][:n], y[::inc][:n]
        s, a = orc.ddot_ld(n, x, inc, y, inc)
        assert abs(s - float(np.dot(xs, ys))) <= 4 * n * 2.0 ** -53 * a
        assert abs(orc.dasum_ld(n, x, inc) - float(np.sum(np.abs(xs)))) <= 4 * n * 2.0 ** -53 * np.sum(np.abs(xs))
        assert abs(orc.dnrm2_ld(n, x, inc) - float(np.linalg.norm(xs))) <= 4 * n * 2.0 ** -53 * np.linalg.norm(xs)
        assert orc.idamax_brute(n, x, inc) == int(np.argmax(np.abs(xs)))
