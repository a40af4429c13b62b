"""GPU parity of ssyr2k, ssymm, strmm and strsm through the C ABI, against the
oracle's long-double restatements, under the reference's own metrics:

  * ssyr2k (tests/ssyr2k/helpers.js): |C - C_ref| <= eps ((k+3)|alpha| d1 +
    (k+2)|alpha| d2 + 3|beta||C_in|) on the triangle, d1 / d2 the two
    products' sum |a b|; the other triangle bit-identical.
  * ssymm (tests/ssymm/helpers.js): eps ((order+1)|alpha| sum|S B| + |beta||C_in|).
  * strmm (tests/strmm/helpers.js): eps (order+1) |alpha| sum|op(A) B|.
  * strsm (tests/strsm/helpers.js): backward residual
    |op(A) X - alpha B| <= eps (order+1) sum|op(A)||X| (factor <= 1 here;
    the reference allows 5 for its explicit block inverses).
eps = 2^-23. Cases are written in the reference's terms (layout, side, uplo,
trans, diag) and mapped onto the column-major C ABI the way the JS layer maps
them (tests/refcases.py); ld padding must come back bit-identical.
"""
import itertools

import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, bits_equal

pytestmark = pytest.mark.gpu

F32 = np.float32


def up(ctx, a):
    a = np.asarray(a, F32)
    return ctx.upload(a if a.size else np.zeros(1, F32))


def factor(got, ref, bound, idx):
    got = np.asarray(got, np.float64)[idx]
    ref = np.asarray(ref, np.float64)[idx]
    bound = np.asarray(bound, np.float64)[idx]
    err = np.abs(got - ref)
    with np.errstate(invalid="ignore", divide="ignore"):
        f = np.where(bound == 0, np.where(err == 0, 0.0, np.inf), err / np.where(bound == 0, 1, bound))
    return float(f.max()) if f.size else 0.0


def c_term(beta, C):
    """|beta| |C_in|, zero when beta = 0 (C is not read then, NaN included)."""
    if beta == 0:
        return np.zeros(len(C))
    return abs(beta) * np.abs(np.asarray(C, np.float64))


def region(m, n, ld, uplo=0):
    """Indices of the m x n (uplo part of the) column-major matrix."""
    i = np.arange(m)[:, None]
    j = np.arange(n)[None, :]
    mask = np.ones((m, n), bool) if uplo == 0 else ((i >= j) if uplo == 1 else (i <= j))
    return (i + j * ld)[mask]


def outside(total, idx):
    keep = np.ones(total, bool)
    keep[idx] = False
    return keep


# ------------------------------------------------------------------ runners
def check_syr2k(ctx, call):
    uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc = call
    dC = up(ctx, C)
    ctx.ssyr2k(uplo, trans, n, k, alpha, up(ctx, A), lda, up(ctx, B), ldb, beta, dC, ldc)
    got = dC.to_host()
    ref, d1, d2 = orc.ssyr2k_ld(*call)
    idx = region(n, n, ldc, uplo)
    bound = EPS32 * ((k + 3) * abs(alpha) * d1 + (k + 2) * abs(alpha) * d2 + 3 * c_term(beta, C))
    assert factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F32)[keep])
    return got


def check_symm(ctx, call):
    side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc = call
    dC = up(ctx, C)
    ctx.ssymm(side, uplo, m, n, alpha, up(ctx, A), lda, up(ctx, B), ldb, beta, dC, ldc)
    got = dC.to_host()
    ref, ad = orc.ssymm_ld(*call)
    order = m if side == 1 else n
    idx = region(m, n, ldc)
    bound = EPS32 * ((order + 1) * abs(alpha) * ad + c_term(beta, C))
    assert factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F32)[keep])
    return got


def check_trmm(ctx, call):
    side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb = call
    dB = up(ctx, B)
    ctx.strmm(side, uplo, trans, unit, m, n, alpha, up(ctx, A), lda, dB, ldb)
    got = dB.to_host()
    ref, ad = orc.strmm_ld(*call)
    order = m if side == 1 else n
    idx = region(m, n, ldb)
    assert factor(got, ref, EPS32 * (order + 1) * abs(alpha) * ad, idx) <= 1
    keep = outside(len(B), idx)
    assert bits_equal(got[keep], np.asarray(B, F32)[keep])
    return got


def residual_factor(X, call):
    """tests/strsm/helpers.js backwardResidualFactor on the column-major X."""
    side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb = call
    order = m if side == 1 else n
    T = rc.dense_tri(np.asarray(A, F32), order, lda, uplo, trans, unit)
    Xd = rc.dense_op(X, m, n, ldb, 0)
    Bd = rc.dense_op(np.asarray(B, F32), m, n, ldb, 0)
    prod = T @ Xd if side == 1 else Xd @ T
    absprod = np.abs(T) @ np.abs(Xd) if side == 1 else np.abs(Xd) @ np.abs(T)
    rhs = 0.0 if alpha == 0 else alpha * Bd
    err = np.abs(prod - rhs)
    bound = EPS32 * (order + 1) * absprod
    with np.errstate(invalid="ignore", divide="ignore"):
        f = np.where(bound == 0, np.where(err == 0, 0.0, np.inf), err / np.where(bound == 0, 1, bound))
    return float(f.max()) if f.size else 0.0


def run_trsm(ctx, call):
    side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb = call
    dB = up(ctx, B)
    ctx.strsm(side, uplo, trans, unit, m, n, alpha, up(ctx, A), lda, dB, ldb)
    return dB.to_host()


def check_trsm(ctx, call, threshold=1.0):
    side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb = call
    got = run_trsm(ctx, call)
    assert residual_factor(got, call) <= threshold
    keep = outside(len(B), region(m, n, ldb))
    assert bits_equal(got[keep], np.asarray(B, F32)[keep])
    return got


# ------------------------------------------------------------ edge cases
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases(ctx, cm):
    for c in rc.load("ssyr2k", cm):
        check_syr2k(ctx, rc.syr2k_call(c))
    for c in rc.load("ssymm", cm):
        check_symm(ctx, rc.symm_call(c))
    for c in rc.load("strmm", cm):
        check_trmm(ctx, rc.tri_call(c))
    for c in rc.load("strsm", cm):
        call = rc.tri_call(c)
        got = check_trsm(ctx, call)
        # the fixtures are small and well conditioned: also close to the oracle
        ref = orc.strsm_ld(*call)
        idx = region(call[4], call[5], call[10])
        assert np.allclose(got[idx], ref[idx], rtol=1e-6, atol=1e-6), c["label"]


# ------------------------------------------------------------ ssyr2k
def syr2k_case(layout, N, K, uplo, trans, alpha=1.5, beta=0.5, seeds=(71, 72, 73)):
    # tests/ssyr2k/src/test.ssyr2k.js:167-231: op(A) N x K, ld = stored columns
    aR, aC = (N, K) if trans == "no-transpose" else (K, N)
    ld = aR if layout == "column-major" else aC
    return dict(layout=layout, uplo=uplo, trans=trans, n=N, k=K, alpha=alpha, beta=beta,
                A=orc.random_f32(aR * aC, -1, 1, seeds[0]), lda=ld,
                B=orc.random_f32(aR * aC, -1, 1, seeds[1]), ldb=ld,
                C=orc.random_f32(N * N, -1, 1, seeds[2]), ldc=N)


@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("N", [150, 400])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
def test_ssyr2k_multi_tile(ctx, layout, N, uplo, trans):
    check_syr2k(ctx, rc.syr2k_call(syr2k_case(layout, N, 9, uplo, trans)))


@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_ssyr2k_k0_and_alpha0(ctx, uplo):
    # test.ssyr2k.js:233-287 (k = 0: beta*C on the triangle) and 332-376
    # (alpha = 0 with NaN / Inf in A and B, NaN in C when beta = 0)
    for n in (7, 300):
        for beta in (0.0, 0.5):
            c = syr2k_case("row-major", n, n, uplo, "no-transpose", alpha=0.0, beta=beta, seeds=(1, 2, 3))
            c["A"][1 * n + 2], c["A"][3 * n + 0], c["B"][2 * n + 3] = np.nan, -np.inf, np.inf
            if beta == 0:
                c["C"][4 * n + 4] = np.nan
            got = check_syr2k(ctx, rc.syr2k_call(c))
            assert np.all(np.isfinite(got))
    c = syr2k_case("column-major", 64, 0, uplo, "no-transpose")
    check_syr2k(ctx, rc.syr2k_call(c))


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_ssyr2k_large_tier_padded(ctx, uplo, trans):
    n, k = 1100, 333
    lda = (k if trans else n) + 3
    ldb = (k if trans else n) + 1
    ldc = n + 2
    cols = n if trans else k
    call = (uplo, trans, n, k, 0.75, orc.random_f32(lda * cols, -1, 1, 5), lda,
            orc.random_f32(ldb * cols, -1, 1, 6), ldb, -1.25, orc.random_f32(ldc * n, -1, 1, 7), ldc)
    check_syr2k(ctx, call)


def syr2k_sampled(ctx, uplo, trans, n, k, alpha, beta, ld, ldc, seed, dt=np.float32):
    """ssyr2k / dsyr2k with lda == ldb, the shape of the one-launch path
    (both products over one two-part k range when k is whole k-tiles),
    with inputs generated on the device. Sampled columns of the triangle
    are checked against float64 products under the reference's bound, and
    C's other triangle and ld padding must come back bit-identical."""
    from tests.helpers import EPS_DD

    f64 = dt == np.float64
    cols = n if trans else k
    A, B = ctx.empty(ld * cols, dt), ctx.empty(ld * cols, dt)
    C = ctx.empty(ldc * n, dt)
    try:
        for i, X in enumerate((A, B, C)):
            ctx.fill_uniform(X, -1.0, 1.0, seed + i)
        ctx.synchronize()
        a, b, cin = A.to_host(), B.to_host(), C.to_host()
        (ctx.dsyr2k if f64 else ctx.ssyr2k)(uplo, trans, n, k, alpha, A, ld, B, ld, beta, C, ldc)
        got = C.to_host()
    finally:
        for X in (A, B):
            X.free()
        C.free()

    def op(x):  # op(X) as n x k float64
        return (x.reshape(n, ld)[:, :k] if trans else x.reshape(k, ld)[:, :n].T).astype(np.float64)

    oa, ob = op(a), op(b)
    keep = np.ones(len(cin), bool)
    keep[region(n, n, ldc, uplo)] = False
    assert bits_equal(got[keep], cin[keep]), "other triangle or ld padding written"
    rng = np.random.default_rng(seed)
    sel = np.unique(np.concatenate([[0, n - 1, n // 2, min(n - 1, 128), min(n - 1, 127)],
                                    rng.integers(0, n, 20)]))
    eps, c1, c2, c3 = (EPS_DD, 2, 1, 2) if f64 else (EPS32, 3, 2, 3)
    for j in sel:
        rows = np.arange(j, n) if uplo == 1 else np.arange(0, j + 1)
        cj = cin[j * ldc + rows].astype(np.float64)
        ref = alpha * (oa[rows] @ ob[j] + ob[rows] @ oa[j]) + beta * cj
        d1 = np.abs(oa[rows]) @ np.abs(ob[j])
        d2 = np.abs(ob[rows]) @ np.abs(oa[j])
        bound = eps * ((k + c1) * abs(alpha) * d1 + (k + c2) * abs(alpha) * d2 + c3 * abs(beta) * np.abs(cj))
        err = np.abs(got[j * ldc + rows].astype(np.float64) - ref)
        assert np.all(err <= bound), f"column {j}: max err/bound {np.max(err / bound)}"


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("n,k", [(4224, 544), (4100, 320), (1100, 96)])
def test_ssyr2k_one_launch(ctx, uplo, trans, n, k):
    # lda == ldb and k a multiple of 32: one launch over (A, B) then (B, A).
    # 4224 / 544: 561 tiles of 128 on the 128 tier, a split-k tail whose
    # k-slices straddle the switch from (A, B) to (B, A) (k-tile 17 of 34);
    # 4100 / 320: 561 tiles of 128 with edge tiles (no split: 20 k-tiles);
    # 1100 / 96: 64 tier, edge tiles
    print(f"ssyr2k one launch uplo={uplo} trans={trans} n={n} k={k}", flush=True)
    ld = (k if trans else n) + 4
    syr2k_sampled(ctx, uplo, trans, n, k, 0.75, -0.5, ld, n + 2, 1000 + n)


# ------------------------------------------------------------ ssymm
def symm_case(layout, side, uplo, N, OTHER, pad, alpha=1.5, beta=0.5, seeds=(91, 92, 93)):
    # tests/ssymm/src/test.ssymm.js:236-297
    m = N if side == "left" else OTHER
    n = OTHER if side == "left" else N
    cm = layout == "column-major"
    LD = (m if cm else n) + pad
    OUTER = n if cm else m
    return dict(layout=layout, side=side, uplo=uplo, m=m, n=n, alpha=alpha, beta=beta,
                A=orc.random_f32(N * N, -1, 1, seeds[0]), lda=N,
                B=orc.random_f32(OUTER * LD, -1, 1, seeds[1]), ldb=LD,
                C=orc.random_f32(OUTER * LD, -1, 1, seeds[2]), ldc=LD)


@pytest.mark.parametrize("N,pad", [(150, 1), (400, 4)])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("side", ["left", "right"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_ssymm_multi_tile(ctx, N, pad, layout, side, uplo):
    check_symm(ctx, rc.symm_call(symm_case(layout, side, uplo, N, 72, pad)))


@pytest.mark.parametrize("side", ["left", "right"])
def test_ssymm_alpha0_and_unread_triangle(ctx, side):
    # test.ssymm.js:342-385; plus NaN in the unstored triangle never read
    for n in (7, 300):
        for beta in (0.0, 0.5):
            c = symm_case("row-major", side, "lower", n, n, 0, alpha=0.0, beta=beta, seeds=(1, 2, 3))
            c["A"][3 * n + 1], c["B"][2 * n + 3] = np.nan, np.inf
            if beta == 0:
                c["C"][4 * n + 4] = np.nan
            assert np.all(np.isfinite(check_symm(ctx, rc.symm_call(c))))
    c = symm_case("column-major", side, "lower", 300, 130, 3)
    c["A"][0 + 299 * 300] = np.nan  # column-major (0, 299): upper, unstored
    assert np.all(np.isfinite(check_symm(ctx, rc.symm_call(c))))


@pytest.mark.parametrize("side", [1, 2])
@pytest.mark.parametrize("uplo", [1, 2])
def test_ssymm_large(ctx, side, uplo):
    m, n = (1500, 700) if side == 1 else (700, 1500)
    order = m if side == 1 else n
    lda, ldb, ldc = order + 1, m + 4, m + 3
    call = (side, uplo, m, n, 1.0, orc.random_f32(lda * order, -1, 1, 8), lda,
            orc.random_f32(ldb * n, -1, 1, 9), ldb, 0.25, orc.random_f32(ldc * n, -1, 1, 10), ldc)
    check_symm(ctx, call)


# ------------------------------------------------------------ strmm
def tri_case(layout, side, uplo, transA, diag, N, OTHER, pad, alpha=1.5, seeds=(81, 82)):
    # tests/strmm/src/test.strmm.js:230-294 (and strsm's 273-416)
    m = N if side == "left" else OTHER
    n = OTHER if side == "left" else N
    cm = layout == "column-major"
    LD = (m if cm else n) + pad
    OUTER = n if cm else m
    return dict(layout=layout, side=side, uplo=uplo, transA=transA, diag=diag, m=m, n=n,
                alpha=alpha, A=orc.random_f32(N * N, -1, 1, seeds[0]), lda=N,
                B=orc.random_f32(OUTER * LD, -1, 1, seeds[1]), ldb=LD)


COMBOS = list(itertools.product(["row-major", "column-major"], ["left", "right"], ["lower", "upper"],
                                ["no-transpose", "transpose"]))


@pytest.mark.parametrize("N,pad", [(150, 1), (400, 4)])
@pytest.mark.parametrize("layout,side,uplo,transA", COMBOS)
def test_strmm_multi_tile(ctx, N, pad, layout, side, uplo, transA):
    diag = "unit" if transA == "transpose" else "non-unit"
    check_trmm(ctx, rc.tri_call(tri_case(layout, side, uplo, transA, diag, N, 72, pad)))


@pytest.mark.parametrize("side", ["left", "right"])
def test_strmm_alpha0(ctx, side):
    # test.strmm.js:336-374: B becomes zero, NaN / Inf in A and B never read
    for n in (7, 300):
        c = tri_case("row-major", side, "lower", "no-transpose", "non-unit", n, n, 0, alpha=0.0,
                     seeds=(1, 2))
        c["A"][3 * n + 1], c["B"][2 * n + 3], c["B"][0] = np.nan, np.inf, np.nan
        got = check_trmm(ctx, rc.tri_call(c))
        assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
def test_strmm_large_band(ctx, side, uplo, trans):
    # 128-tiles over a 1500-order triangle: the k band of every tile row
    m, n = (1500, 900) if side == 1 else (900, 1500)
    order = m if side == 1 else n
    lda, ldb = order + 2, m + 1
    call = (side, uplo, trans, 0, m, n, 0.5, orc.random_f32(lda * order, -1, 1, 11), lda,
            orc.random_f32(ldb * n, -1, 1, 12), ldb)
    check_trmm(ctx, call)


def trmm_sampled(ctx, side, uplo, trans, unit, m, n, alpha, lda, ldb, seed, dt=np.float32):
    """strmm / dtrmm on device-generated inputs. The unreferenced triangle
    of A holds NaN, and its diagonal too for a unit triangle, so any of it
    reaching the product shows. Sampled columns against float64 under the
    reference's bound; B's ld padding bit-identical."""
    from tests.helpers import EPS_DD

    order = m if side == 1 else n
    A, B = ctx.empty(lda * order, dt), ctx.empty(ldb * n, dt)
    try:
        ctx.fill_uniform(A, -1.0, 1.0, seed)
        ctx.fill_uniform(B, -1.0, 1.0, seed + 1)
        ctx.synchronize()
        a = A.to_host()
        M = a.reshape(order, lda)[:, :order].T.astype(np.float64)  # M[i, j] = A(i, j)
        i, j = np.arange(order)[:, None], np.arange(order)[None, :]
        stored = (i > j) if uplo == 1 else (i < j)
        if not unit:
            stored = stored | (i == j)
        poison = a.reshape(order, lda).copy()
        poison[:, :order][~stored.T] = np.nan  # (column-major: row index j of the view = column)
        ctx.h2d(A.ptr, poison.reshape(-1))
        bin_ = B.to_host()
        fn = ctx.dtrmm if dt == np.float64 else ctx.strmm
        fn(side, uplo, trans, 1 if unit else 0, m, n, alpha, A, lda, B, ldb)
        got = B.to_host()
    finally:
        A.free()
        B.free()
    T = np.where(stored, M, 0.0)
    if unit:
        T[np.arange(order), np.arange(order)] = 1.0
    opA = T.T if trans else T
    Bm = bin_.reshape(n, ldb)[:, :m].T.astype(np.float64)
    pad = np.ones((n, ldb), bool)
    pad[:, :m] = False
    assert bits_equal(got.reshape(n, ldb)[pad], bin_.reshape(n, ldb)[pad])
    eps = EPS_DD if dt == np.float64 else EPS32
    rng = np.random.default_rng(seed)
    cols = np.unique(np.concatenate([[0, n - 1, min(n - 1, 127), min(n - 1, 128)], rng.integers(0, n, 12)]))
    G = got.reshape(n, ldb)[:, :m].T.astype(np.float64)
    for c in cols:
        if side == 1:
            ref = alpha * (opA @ Bm[:, c])
            ad = abs(alpha) * (np.abs(opA) @ np.abs(Bm[:, c]))
        else:
            ref = alpha * (Bm @ opA[:, c])
            ad = abs(alpha) * (np.abs(Bm) @ np.abs(opA[:, c]))
        assert np.all(np.isfinite(G[:, c])), f"column {c}: the unreferenced triangle leaked"
        assert np.all(np.abs(G[:, c] - ref) <= eps * (order + 2) * ad), f"column {c}"


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
@pytest.mark.parametrize("unit", [0, 1])
@pytest.mark.parametrize("dims", [(3000, 2900), (700, 260)])
def test_strmm_large_unreferenced_nan(ctx, side, uplo, trans, unit, dims):
    # 3000 x 2900 puts the banded launch on 128-tiles with edge tiles,
    # 700 x 260 on 64-tiles; NaN wherever A is not referenced
    m, n = dims
    order = m if side == 1 else n
    print(f"strmm side={side} uplo={uplo} trans={trans} unit={unit} {m}x{n}", flush=True)
    trmm_sampled(ctx, side, uplo, trans, unit, m, n, 0.75, order + 4, m + 3, 77 + order)


# ------------------------------------------------------------ strsm
def well_conditioned(c, N):
    # tests/strsm/src/test.strsm.js:294-296: off-diagonals in [-1/N, 1/N), diagonal 2
    A = orc.random_f32(N * N, -1.0 / N, 1.0 / N, 121)
    for i in range(N):
        A[i * N + i] = 2
    c["A"] = A
    return c


@pytest.mark.parametrize("N,OTHER", [(64, 70), (37, 7), (1, 7)])
@pytest.mark.parametrize("layout,side,uplo,transA", COMBOS)
def test_strsm_single_block(ctx, N, OTHER, layout, side, uplo, transA):
    # test.strsm.js:273-347: one substitution block, alpha 1.5, ld padding 3
    diag = "unit" if uplo == "upper" else "non-unit"
    c = well_conditioned(tri_case(layout, side, uplo, transA, diag, N, OTHER, 3, seeds=(121, 122)), N)
    check_trsm(ctx, rc.tri_call(c))


@pytest.mark.parametrize("N,OTHER,pad", [(150, 70, 1), (600, 200, 4)])
@pytest.mark.parametrize("layout,side,uplo,transA", COMBOS)
def test_strsm_many_block(ctx, N, OTHER, pad, layout, side, uplo, transA):
    # test.strsm.js:349-415: several blocks, in-place GEMM updates
    diag = "unit" if transA == "transpose" else "non-unit"
    c = well_conditioned(tri_case(layout, side, uplo, transA, diag, N, OTHER, pad, seeds=(121, 122)), N)
    check_trsm(ctx, rc.tri_call(c))


@pytest.mark.parametrize("side,uplo", [("left", "lower"), ("left", "upper"), ("right", "lower")])
def test_strsm_more_than_one_block(ctx, side, uplo):
    # test.strsm.js:467-522: order 70, 5 right-hand sides, entries in [-0.5, 0.5]
    order, other = 70, 5
    m, n = (order, other) if side == "left" else (other, order)
    A = orc.random_f32(order * order, -0.5, 0.5, 3)
    for i in range(order):
        A[i * order + i] = np.float32(0.5) + np.abs(A[i * order + i])  # diagonal away from 0
    c = dict(layout="row-major", side=side, uplo=uplo, transA="no-transpose", diag="non-unit",
             m=m, n=n, alpha=1.0, A=A, lda=order, B=orc.random_f32(m * n, -1, 1, 4), ldb=n)
    check_trsm(ctx, rc.tri_call(c))


def test_strsm_alpha0_literal_zero(ctx):
    # test.strsm.js:173-199
    c = dict(layout="row-major", side="left", uplo="lower", transA="no-transpose", diag="non-unit",
             m=2, n=2, alpha=0.0, A=np.array([1, 0, 1, 1], F32), lda=2,
             B=np.array([np.inf, np.nan, 3, 4], F32), ldb=2)
    assert np.array_equal(run_trsm(ctx, rc.tri_call(c)), np.zeros(4, F32))


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("transA", ["no-transpose", "transpose"])
@pytest.mark.parametrize("m", [7, 600])
@pytest.mark.parametrize("where", ["B early", "B mid", "B late", "A"])
def test_strsm_ieee_specials(ctx, uplo, transA, m, where):
    # test.strsm.js:524-578: Inf / NaN land where substitution puts them; NaN
    # in the unreferenced triangle is never read. The oracle substitutes in
    # long double, so the non-finite pattern must match exactly and finite
    # values within 1e-4 relative.
    n = 5
    at = lambda r, cc, ld: r * ld + cc  # row-major
    A = orc.random_f32(m * m, -1, 1, 1)
    for i in range(m):
        A[at(i, i, m)] += m + 4
    A[at(1, 4, m) if uplo == "lower" else at(4, 1, m)] = np.nan
    B = orc.random_f32(m * n, -1, 1, 2)
    if where == "B early":
        B[at(1, 2, n)] = np.inf
    elif where == "B mid":
        B[at(m // 2, 0, n)] = np.inf
    elif where == "B late":
        B[at(m - 2, 4, n)] = -np.inf
    else:
        A[at(m - 1, 2, m) if uplo == "lower" else at(2, m - 1, m)] = np.inf
    c = dict(layout="row-major", side="left", uplo=uplo, transA=transA, diag="non-unit", m=m, n=n,
             alpha=1.0, A=A, lda=m, B=B, ldb=n)
    call = rc.tri_call(c)
    got = run_trsm(ctx, call).astype(np.float64)
    ref = orc.strsm_ld(*call)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))
    assert np.array_equal(np.sign(got[np.isinf(got)]), np.sign(ref[np.isinf(ref)]))
    fin = np.isfinite(ref)
    assert np.allclose(got[fin], ref[fin], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
def test_strsm_large_round_trip(ctx, side, uplo, trans):
    # 2000-order solves (five recursion levels, 128-tier updates with split-k
    # tails): the residual bound on sampled right-hand sides, and strmm of the
    # solution gives back alpha * B
    order, other = 2000, 300
    m, n = (order, other) if side == 1 else (other, order)
    lda, ldb = order + 1, m + 3
    A = orc.random_f32(lda * order, -1.0 / order, 1.0 / order, 13)
    A[np.arange(order) * (lda + 1)] = 2.0
    B = orc.random_f32(ldb * n, -1, 1, 14)
    call = (side, uplo, trans, 0, m, n, 1.5, A, lda, B, ldb)
    X = check_trsm(ctx, call)
    dB = up(ctx, X)
    ctx.strmm(side, uplo, trans, 0, m, n, 1.0, up(ctx, A), lda, dB, ldb)
    back = rc.dense_op(dB.to_host(), m, n, ldb, 0)
    want = 1.5 * rc.dense_op(B, m, n, ldb, 0)
    assert np.max(np.abs(back - want)) <= 1e-4 * np.max(np.abs(want))


@pytest.mark.parametrize("side,uplo,trans", list(itertools.product([1, 2], [1, 2], [0, 1])))
def test_strsm_many_right_hand_sides(ctx, side, uplo, trans):
    # 8200 right-hand sides: 513 groups of 16, the last one padded.
    # Order 300 (diagonal blocks of 256 and 44, a GEMM update between): the
    # residual bound. Order 100 (one padded diagonal block, no GEMM):
    # every right-hand side's solution is bit-equal to solving it among only
    # 100, since a right-hand side's operations do not depend on how many
    # are solved together (each is one column of the MFMA products).
    other = 8200
    for order in (300, 100):
        m, n = (order, other) if side == 1 else (other, order)
        lda, ldb = order + 2, m + 1
        A = orc.random_f32(lda * order, -1.0 / order, 1.0 / order, 15)
        A[np.arange(order) * (lda + 1)] = 2.0
        B = orc.random_f32(ldb * n, -1, 1, 16)
        X = check_trsm(ctx, (side, uplo, trans, 0, m, n, 0.75, A, lda, B, ldb))
    ms, ns = (order, 100) if side == 1 else (100, order)
    Bs = np.asarray(rc.dense_op(B, m, n, ldb, 0)[:ms, :ns], F32).reshape(-1, order="F")
    Xs = run_trsm(ctx, (side, uplo, trans, 0, ms, ns, 0.75, A, lda, Bs, ms))
    Xd = np.asarray(rc.dense_op(X, m, n, ldb, 0)[:ms, :ns], F32).reshape(-1, order="F")
    assert bits_equal(Xs, Xd)


@pytest.mark.parametrize("side,uplo,trans", [(1, 1, 0), (1, 2, 1), (2, 1, 1), (2, 2, 0)])
def test_strsm_special_path_matches(ctx, side, uplo, trans):
    # A right-hand side that holds Inf or NaN sends the 16 it is solved with
    # through the substitution that keeps each row as it is solved (the
    # IEEE-special path), from the sub-block where the value appears to the
    # end of its diagonal block. The other right-hand sides of the group
    # must come out bit-equal to a solve without the specials (the regular
    # path), and the poisoned ones non-finite. Order 300: diagonal blocks of
    # frame rows [0, 256) and [256, 300), the Inf at frame row 100, the NaN
    # at 270 (one in each block, whichever way the solve runs); 40
    # right-hand sides = groups of 16, 16 and 8.
    order, other = 300, 40
    m, n = (order, other) if side == 1 else (other, order)
    lda, ldb = order + 3, m + 2
    A = orc.random_f32(lda * order, -1.0 / order, 1.0 / order, 21)
    A[np.arange(order) * (lda + 1)] = 2.0
    B = orc.random_f32(ldb * n, -1, 1, 22)
    # frame row f of right-hand side r sits at B(f, r) (left) or B(r, f) (right)
    at = (lambda f, r: f + r * ldb) if side == 1 else (lambda f, r: r + f * ldb)
    Bs = B.copy()
    Bs[at(100, 5)] = np.inf
    Bs[at(270, 37)] = np.nan
    call = lambda Bx: (side, uplo, trans, 0, m, n, 0.75, A, lda, Bx, ldb)
    X = run_trsm(ctx, call(B))
    Xs = run_trsm(ctx, call(Bs))
    rhs = lambda Xa, r: np.array([Xa[at(f, r)] for f in range(order)], F32)
    for r in range(other):
        if r in (5, 37):
            assert not np.all(np.isfinite(rhs(Xs, r)))
        else:
            assert bits_equal(rhs(X, r), rhs(Xs, r)), r


def _blocks_of_condition(order, lda, seed, weak, scale):
    """Column-major A (lda x order): off-diagonals in [-1/order, 1/order),
    diagonal 2, except that every 256-order diagonal block listed in `weak`
    holds off-diagonals in [-scale, scale) and a unit diagonal. With scale
    0.1 such a block's condition number ||M||_1 ||M^-1||_1 is about 260, far
    above what the inverse path accepts (16), with every entry of its inverse
    still of order 1; with 0.02 it is about 14, just below."""
    A = orc.random_f32(lda * order, -1.0 / order, 1.0 / order, seed)
    A[np.arange(order) * (lda + 1)] = 2.0
    W = orc.random_f32(256 * 256, -scale, scale, seed + 1)
    for b in weak:
        lo = 256 * b
        nb = min(256, order - lo)
        for j in range(nb):
            col = (lo + j) * lda + lo
            A[col:col + nb] = W[j * 256:j * 256 + nb]
            A[col + j] = 1.0
    return A


@pytest.mark.parametrize("weak,scale", [((1,), 0.1), ((0, 2), 0.1), ((0, 1, 2), 0.02), ((), 0.1)])
@pytest.mark.parametrize("side,uplo,trans", [(1, 1, 0), (1, 2, 1), (2, 1, 1), (2, 2, 0)])
def test_strsm_node_path_block_conditions(ctx, weak, scale, side, uplo, trans):
    # Order 700: nodes [0, 512) (two diagonal blocks, the inverse path with
    # its coupling block) and [512, 700) (one partial block). A diagonal
    # block whose condition estimate exceeds the inverse path's limit is
    # solved by substitution, the others by their inverses, in either solve
    # direction and on either side; the backward residual bound holds
    # throughout (ill-conditioned blocks included) and ld padding stays
    # untouched. alpha 1.25 exercises the scaling on both paths.
    order, other = 700, 40
    m, n = (order, other) if side == 1 else (other, order)
    lda, ldb = order + 3, m + 2
    A = _blocks_of_condition(order, lda, 131, weak, scale)
    B = orc.random_f32(ldb * n, -1, 1, 132)
    check_trsm(ctx, (side, uplo, trans, 0, m, n, 1.25, A, lda, B, ldb))


@pytest.mark.parametrize("side", [1, 2])
def test_strsm_node_path_rhs_independent_of_batch(ctx, side):
    # Order 600 (the node path), a mix of blocks solved by inverse and by
    # substitution: each right-hand side's solution is bit-equal to solving
    # it alone (one right-hand side per call), so neither path mixes
    # right-hand sides or depends on how many are solved together.
    order, other = 600, 21
    m, n = (order, other) if side == 1 else (other, order)
    lda, ldb = order + 1, m
    A = _blocks_of_condition(order, lda, 141, (1,), 0.1)
    B = orc.random_f32(ldb * n, -1, 1, 142)
    X = run_trsm(ctx, (side, 1, 0, 0, m, n, 0.5, A, lda, B, ldb))
    for r in (0, 7, 20):
        if side == 1:
            Br = np.asarray(B, F32)[r * ldb:r * ldb + order]
            Xr = run_trsm(ctx, (side, 1, 0, 0, order, 1, 0.5, A, lda, Br, order))
            assert bits_equal(Xr, np.asarray(X, F32)[r * ldb:r * ldb + order]), r
        else:
            Br = np.asarray(B, F32)[r::ldb][:order]
            Xr = run_trsm(ctx, (side, 1, 0, 0, 1, order, 0.5, A, lda, Br, 1))
            assert bits_equal(Xr, np.asarray(X, F32)[r::ldb][:order]), r


# ------------------------------------------- operands of different storage orders
def _cm_transpose(X, rows, cols, ld):
    """Column-major rows x cols (leading dimension ld) -> its transpose as a
    dense column-major cols x rows array (leading dimension cols)."""
    M = np.asarray(X, F32)[: ld * cols].reshape(cols, ld)[:, :rows]  # M[j, i] = X(i, j)
    return np.ascontiguousarray(M.T).reshape(-1)  # X^T(j, i) = X(i, j) at j + i*cols


@pytest.mark.parametrize("side", [1, 2])
@pytest.mark.parametrize("uplo", [1, 2])
def test_ssymm_b_other_storage_order(ctx, side, uplo):
    # wgblas accepts a B whose storage order differs from C's
    # (src/ssymm/ssymm.mjs:85-87, 149-163): in C's column-major frame that B
    # is op(B) = B^T of its memory, stored n x m
    m, n = (300, 170) if side == 1 else (170, 300)
    order = m if side == 1 else n
    lda, ldb_t, ldc = order + 2, n + 3, m + 1
    A = orc.random_f32(lda * order, -1, 1, 61)
    Bt = orc.random_f32(ldb_t * m, -1, 1, 62)  # n x m stored, op(B) = its transpose
    C = orc.random_f32(ldc * n, -1, 1, 63)
    dC = up(ctx, C)
    ctx.ssymm(side, uplo, m, n, 1.25, up(ctx, A), lda, up(ctx, Bt), ldb_t, 0.5, dC, ldc, transB=1)
    got = dC.to_host()
    B = _cm_transpose(Bt, n, m, ldb_t)  # m x n, ld m
    ref, ad = orc.ssymm_ld(side, uplo, m, n, 1.25, A, lda, B, m, 0.5, C, ldc)
    idx = region(m, n, ldc)
    bound = EPS32 * ((order + 1) * 1.25 * ad + c_term(0.5, C))
    assert factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F32)[keep])


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_ssyr2k_operands_of_different_storage_orders(ctx, uplo, ta, tb):
    # GpuMatrix A and B of different layouts reach one wgb_ssyr2k call with a
    # flag per operand; the oracle sees B converted to A's orientation
    n, k = 333, 150
    lda = (k if ta else n) + 2
    ldb = (k if tb else n) + 1
    ldc = n + 4
    A = orc.random_f32(lda * (n if ta else k), -1, 1, 64)
    B = orc.random_f32(ldb * (n if tb else k), -1, 1, 65)
    C = orc.random_f32(ldc * n, -1, 1, 66)
    dC = up(ctx, C)
    ctx.ssyr2k(uplo, ta, n, k, 0.75, up(ctx, A), lda, up(ctx, B), ldb, -0.5, dC, ldc, transB=tb)
    got = dC.to_host()
    rows_b, cols_b = (k, n) if tb else (n, k)
    Bc = _cm_transpose(B, rows_b, cols_b, ldb)  # the other orientation, ld = cols_b
    call = (uplo, ta, n, k, 0.75, A, lda, Bc, cols_b, -0.5, C, ldc)
    ref, d1, d2 = orc.ssyr2k_ld(*call)
    idx = region(n, n, ldc, uplo)
    bound = EPS32 * ((k + 3) * 0.75 * d1 + (k + 2) * 0.75 * d2 + 3 * c_term(-0.5, C))
    assert factor(got, ref, bound, idx) <= 1
    keep = outside(len(C), idx)
    assert bits_equal(got[keep], np.asarray(C, F32)[keep])
