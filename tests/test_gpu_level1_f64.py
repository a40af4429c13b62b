"""GPU parity of the fp64 level-1 reductions (ddot, dasum, dnrm2, idamax)
through the C ABI.

Bars, from wgblas's own tests of these routines (which compare its
double-double results with stdlib's float64 ones): ddot within
n * 2^-48 * sum|x y| (tests/ddot/helpers.js), dasum within 64 ULP
(tests/dasum/src/test.dasum.js:20), dnrm2 within 10 * 2^-48 relative
(tests/dnrm2/helpers.js, test.dnrm2.js:28), idamax exact. The exact values
come from the oracle's long-double sums; past the reference's fixture sizes
(n <= 50) dasum is held to the float64 forward bound n * 2^-53 * sum|x|.
ddot is also held to a bar 16x tighter than the reference's.
The reference's "f32 exponent range" regressions describe double-double's
limits and have no counterpart here (values stay finite as in real f64).
"""
import math

import numpy as np
import pytest

from oracle import orc
from tests import refcases
from tests.test_oracle import DNRM2_EXPECT, IDAMAX_EXPECT

pytestmark = pytest.mark.gpu

EPS_DD = 2.0 ** -48
TIGHT = 1.0 / 16


def up(ctx, host):
    return ctx.upload(np.ascontiguousarray(host, np.float64))


def ulps64(a, b):
    if a == b or (math.isnan(a) and math.isnan(b)):
        return 0
    ia = np.array(a, np.float64).view(np.int64)
    ib = np.array(b, np.float64).view(np.int64)
    return abs(int(ia) - int(ib))


def check_ddot(ctx, n, x, incx, y, incy, label=""):
    got = ctx.ddot(n, up(ctx, x), incx, up(ctx, y), incy)
    want, sum_abs = orc.ddot_ld(n, x, incx, y, incy)
    bound = n * EPS_DD * sum_abs
    err = abs(got - want)
    assert err <= bound if bound > 0 else got == want, label
    assert err <= TIGHT * bound if bound > 0 else True, label
    return got


def check_dasum(ctx, n, x, incx, label=""):
    got = ctx.dasum(n, up(ctx, x), incx)
    want = orc.dasum_ld(n, x, incx)
    if n <= 50:
        assert ulps64(got, want) <= 64, label
    else:
        assert abs(got - want) <= n * 2.0 ** -53 * want, label
    return got


def check_dnrm2(ctx, n, x, incx, label=""):
    got = ctx.dnrm2(n, up(ctx, x), incx)
    want = orc.dnrm2_ld(n, x, incx)
    err = abs(got - want)
    assert err <= 10 * EPS_DD * abs(want) or err == 0, f"{label}: {got} vs {want}"
    return got


# ------------------------------------------------------------ edge cases
def test_ddot_edge_cases(ctx):
    for c in refcases.load("ddot"):
        check_ddot(ctx, c["n"], np.array(c["x"], np.float64), c["incx"], np.array(c["y"], np.float64),
                   c["incy"], c["label"])


def test_dasum_edge_cases(ctx):
    for c in refcases.load("dasum"):
        check_dasum(ctx, c["n"], np.array(c["x"], np.float64), c["incx"], c["label"])


def test_dnrm2_edge_cases(ctx):
    for c, want in zip(refcases.load("dnrm2"), DNRM2_EXPECT):
        got = check_dnrm2(ctx, c["n"], np.array(c["x"], np.float64), c["incx"], c["label"])
        if want is not None and want in (0.0, 1.0, 5.0):
            assert got == want, c["label"]


def test_idamax_edge_cases_exact(ctx):
    for c, want in zip(refcases.load("idamax"), IDAMAX_EXPECT):
        assert ctx.idamax(c["n"], up(ctx, np.array(c["x"], np.float64)), c["incx"]) == want, c["label"]


# ------------------------------------------------------ reference regressions
def test_zero_dimension(ctx):
    # test.{ddot,dasum,dnrm2,idamax}.js "zero-dimension": n = 0 gives 0 / -1
    x = up(ctx, orc.random_f64(8, -1, 1, 300))
    assert ctx.ddot(0, x, 1, x, 1) == 0.0
    assert ctx.dasum(0, x, 1) == 0.0
    assert ctx.dnrm2(0, x, 1) == 0.0
    assert ctx.idamax(0, x, 1) == -1
    assert ctx.idamax(-3, x, 1) == -1
    out = ctx.empty(1, np.float64)
    iout = ctx.empty(1, np.int64)
    ctx.dnrm2_dev(0, x, 1, out)
    ctx.idamax_dev(0, x, 1, iout)
    assert out.to_host()[0] == 0.0 and iout.to_host()[0] == -1


@pytest.mark.parametrize("n", [1, 7, 50, 4097, 100003])
@pytest.mark.parametrize("inc", [1, 2, 3, 5])
def test_random_vectors_within_bounds(ctx, n, inc):
    # test.*.js "fixtures": random inputs (here also long and strided)
    rng = np.random.default_rng(n * 10 + inc)
    x = rng.uniform(-1, 1, (n - 1) * inc + 1)
    y = rng.uniform(-1, 1, (n - 1) * inc + 1)
    check_ddot(ctx, n, x, inc, y, inc)
    check_ddot(ctx, n, x, inc, y[: (n - 1) + 1], 1)  # different strides
    check_dasum(ctx, n, x, inc)
    check_dnrm2(ctx, n, x, inc)
    assert ctx.idamax(n, up(ctx, x), inc) == orc.idamax_brute(n, x, inc)


def test_misaligned_unit_stride(ctx):
    # a vector starting 8 bytes into its allocation takes the element path
    n = 10001
    x = orc.random_f64(n + 1, -1, 1, 5)
    y = orc.random_f64(n + 1, -1, 1, 6)
    dx, dy = up(ctx, x), up(ctx, y)
    got = ctx.ddot(n, dx.offset(1), 1, dy.offset(1), 1)
    want, sum_abs = orc.ddot_ld(n, x[1:], 1, y[1:], 1)
    assert abs(got - want) <= TIGHT * n * EPS_DD * sum_abs
    assert ctx.idamax(n, dx.offset(1), 1) == orc.idamax_brute(n, x[1:], 1)


def test_ieee_special_values(ctx):
    # test.ddot.js:127-152, test.dasum.js:105-121, test.dnrm2.js:211-227,
    # test.idamax.js:128-144: Inf and NaN reach the results as in real f64
    for entries, n in (({2: math.inf}, 7), ({3: -math.inf}, 5000), ({2: math.nan}, 7),
                       ({4000: math.nan}, 5000)):
        x = orc.random_f64(n, -1, 1, 1)
        for i, v in entries.items():
            x[i] = v
        dx = up(ctx, x)
        want = float(np.sum(np.abs(x)))
        got = ctx.dasum(n, dx, 1)
        assert (math.isnan(got) and math.isnan(want)) or got == want or abs(got - want) < 1e-9
        d = ctx.ddot(n, dx, 1, dx, 1)
        assert (math.isnan(d) and any(math.isnan(v) for v in entries.values())) or math.isinf(d)
    for entries, n, want in (({2: math.inf}, 7, 2), ({3: -math.inf, 5: math.inf}, 7, 3),
                             ({4000: -math.inf}, 5000, 4000)):
        x = orc.random_f64(n, -1, 1, 1)
        for i, v in entries.items():
            x[i] = v
        assert ctx.idamax(n, up(ctx, x), 1) == want


def test_idamax_nan_handling(ctx):
    # test.idamax.js:97-126
    run = lambda a: ctx.idamax(len(a), up(ctx, np.array(a, np.float64)), 1)
    N, I = math.nan, math.inf
    assert run([1, N, 7, 3]) == 2 and run([1, 2, 3, N]) == 2
    assert run([N, N, N, N]) == 0
    assert run([N, 5, 2, 3]) == 1 and run([N, I, 2, 3]) == 1
    assert run([1, I, 2, 3]) == 1 and run([1, -I, 2, 3]) == 1


def test_idamax_planted_duplicate_max_large(ctx):
    n = 1 << 22
    x = orc.random_f64(n, -1, 1, 9)
    x[n // 3], x[2 * n // 3] = 5.0, -5.0
    assert ctx.idamax(n, up(ctx, x), 1) == n // 3
    assert ctx.idamax(n // 3, up(ctx, x), 3) == orc.idamax_brute(n // 3, x, 3)


DNRM2_REGIMES = [
    ("medium only", lambda i: np.sin(i) * 3),
    ("big + medium", lambda i: np.where(i % 4096 == 7, 1e30 * (1 + np.sin(i) / 3), np.cos(i))),
    ("near f32 max", lambda i: np.where(i % 65536 == 3, 1e37, 1 + np.sin(i) / 7)),
    ("small + medium", lambda i: np.where(i % 1024 == 0, 1e-5 * (1 + np.sin(i) / 5), 1e-25 * (1 + (i % 7) / 3))),
    ("small only", lambda i: 1e-25 * (1 + np.sin(i) / 4)),
    # beyond double-double's range, inside f64's: the LAPACK big / small sums
    ("f64 big", lambda i: np.where(i % 3 == 0, 1e300, 1.0)),
    ("f64 small", lambda i: 1e-300 * (1 + np.sin(i) / 4)),
    ("f64 small + medium", lambda i: np.where(i % 17 == 0, 1e-200, 1e-160)),
]


@pytest.mark.parametrize("label,gen", DNRM2_REGIMES, ids=[r[0] for r in DNRM2_REGIMES])
@pytest.mark.parametrize("inc", [1, 3])
def test_dnrm2_magnitude_regimes(ctx, label, gen, inc):
    # test.dnrm2.js:122-209 (N = 2^18), plus f64-only ranges
    N = 1 << 18
    x = np.zeros((N - 1) * inc + 1)
    x[::inc] = gen(np.arange(N))
    check_dnrm2(ctx, N, x, inc, label)


def test_dnrm2_specials(ctx):
    # test.dnrm2.js:180-208
    N = 1 << 18
    base = lambda s: np.sin(np.arange(N) * s)
    x = base(1)
    x[12345] = math.inf
    assert ctx.dnrm2(N, up(ctx, x), 1) == math.inf
    x = base(2)
    x[54321] = math.nan
    assert math.isnan(ctx.dnrm2(N, up(ctx, x), 1))
    x = base(3)
    x[1], x[2], x[3], x[999] = 1e30, 1e-30, -math.inf, math.nan
    assert math.isnan(ctx.dnrm2(N, up(ctx, x), 1))
    assert ctx.dnrm2(2, up(ctx, np.array([3e300, 4e300])), 1) == 5e300


@pytest.mark.parametrize("inc", [1, 3])
def test_full_size_device_inputs(ctx, inc):
    # 2^27 doubles (the bytes of config 2's 2^28 floats) at unit stride, 2^25
    # at stride 3: device-generated uniform inputs against the oracle
    n = (1 << 27) if inc == 1 else (1 << 25)
    span = (n - 1) * inc + 1
    dx, dy = ctx.empty(span, np.float64), ctx.empty(span, np.float64)
    ctx.fill_uniform(dx, -1, 1, 1)
    ctx.fill_uniform(dy, -1, 1, 2)
    x, y = dx.to_host(), dy.to_host()
    got = ctx.ddot(n, dx, inc, dy, inc)
    want, sum_abs = orc.ddot_ld(n, x, inc, y, inc)
    assert abs(got - want) <= TIGHT * n * EPS_DD * sum_abs
    ga, wa = ctx.dasum(n, dx, inc), orc.dasum_ld(n, x, inc)
    assert abs(ga - wa) <= n * 2.0 ** -53 * wa
    g2, w2 = ctx.dnrm2(n, dx, inc), orc.dnrm2_ld(n, x, inc)
    assert abs(g2 - w2) <= 10 * EPS_DD * w2
    assert ctx.idamax(n, dx, inc) == orc.idamax_brute(n, x, inc)
    dx.free()
    dy.free()
