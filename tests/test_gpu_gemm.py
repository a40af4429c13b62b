"""GPU parity of sgemm / sgemmtr / ssyrk / dgemm through the C ABI.

Every case compares the HIP result with the oracle's long-double GEMM on the
same inputs under the reference's forward-error bound (<= 1), and checks
bit-for-bit that C's ld padding and (sgemmtr/ssyrk) the other triangle are
untouched. The reference's JSON edge cases must match exactly.
"""
import numpy as np
import pytest

from oracle import orc
from tests import refcases
from tests.helpers import EPS32, bits_equal, gemm_forward_factor, untouched_mask

pytestmark = pytest.mark.gpu


def run_gemm(ctx, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, dtype=np.float32,
             syrk=False):
    """Runs the C ABI routine on uploaded copies and returns C (host)."""
    dA = ctx.upload(np.asarray(A, dtype) if np.size(A) else np.zeros(1, dtype))
    dB = dA if syrk else ctx.upload(np.asarray(B, dtype) if np.size(B) else np.zeros(1, dtype))
    dC = ctx.upload(np.asarray(C, dtype))
    if dtype == np.float64 and syrk:
        ctx.dsyrk(uplo, ta, n, k, alpha, dA, lda, beta, dC, ldc)
    elif dtype == np.float64 and uplo:
        ctx.dgemmtr(uplo, ta, tb, m, n, k, alpha, dA, lda, dB, ldb, beta, dC, ldc)
    elif dtype == np.float64:
        ctx.dgemm(ta, tb, m, n, k, alpha, dA, lda, dB, ldb, beta, dC, ldc)
    elif syrk:
        ctx.ssyrk(uplo, ta, n, k, alpha, dA, lda, beta, dC, ldc)
    elif uplo:
        ctx.sgemmtr(uplo, ta, tb, m, n, k, alpha, dA, lda, dB, ldb, beta, dC, ldc)
    else:
        ctx.sgemm(ta, tb, m, n, k, alpha, dA, lda, dB, ldb, beta, dC, ldc)
    out = dC.to_host()
    for d in {id(dA): dA, id(dB): dB, id(dC): dC}.values():
        d.free()
    return out


def check_case(ctx, uplo, ta, tb, m, n, k, alpha, beta, lda, ldb, ldc, seeds=(0, 100, 200),
               dtype=np.float32, syrk=False):
    if syrk:
        tb, ldb = 1 - ta, lda
    a_cols = (m if ta else k)
    b_cols = (k if tb else n)
    gen = orc.random_f64 if dtype == np.float64 else orc.random_f32
    A = gen(max(lda * a_cols, 1), -1, 1, seeds[0])
    B = A if syrk else gen(max(ldb * b_cols, 1), -1, 1, seeds[1])
    C = gen(ldc * n, -1, 1, seeds[2])
    got = run_gemm(ctx, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, dtype, syrk)
    ref, absdot = orc.gemm_ld(uplo, ta, tb, m, n, k, alpha, A.astype(np.float64), lda,
                              B.astype(np.float64), ldb, beta, C.astype(np.float64), ldc)
    fac = gemm_forward_factor(got, ref, absdot, C, m, n, k, alpha, beta, ldc, uplo,
                              dd=dtype == np.float64)
    assert fac <= 1.0, f"forward factor {fac}"
    keep = untouched_mask(m, n, ldc, n, uplo)
    assert bits_equal(got[keep], C[keep]), "C changed outside its m x n part / triangle"
    return got


# ---------------------------------------------------------------- fixtures
@pytest.mark.parametrize("routine", ["sgemm", "sgemmtr", "dgemm", "dgemmtr"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, routine, cm):
    dtype = np.float64 if routine.startswith("d") else np.float32
    for case in refcases.load(routine, cm):
        call = refcases.gemm_call(case, dtype)
        uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc = call
        if routine.startswith("d") and (alpha == 0 or k == 0) and beta == 1:
            continue  # quick return: C is the caller's own buffer, untouched
        got = run_gemm(ctx, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, dtype)
        want = refcases.numpy_gemm(*call).astype(dtype)
        assert np.array_equal(got, want), case["label"]


@pytest.mark.parametrize("routine", ["ssyrk", "dsyrk"])
@pytest.mark.parametrize("cm", [False, True])
def test_syrk_edge_cases_exact(ctx, routine, cm):
    dtype = np.float64 if routine == "dsyrk" else np.float32
    for case in refcases.load(routine, cm):
        uplo, trans, n, k, alpha, A, lda, beta, C, ldc = refcases.syrk_call(case, dtype)
        if routine == "dsyrk" and (alpha == 0 or k == 0) and beta == 1:
            continue  # quick return
        got = run_gemm(ctx, uplo, trans, 0, n, n, k, alpha, A, lda, None, lda, beta, C, ldc,
                       dtype=dtype, syrk=True)
        want = refcases.numpy_gemm(uplo, trans, 1 - trans, n, n, k, alpha, A, lda, A, lda, beta,
                                   C, ldc).astype(dtype)
        assert np.array_equal(got, want), case["label"]


# ------------------------------------------------------- reference regressions
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_large_tile_path_400(ctx, ta, tb):
    # tests/sgemm/src/test.sgemm.js:175-230 (M=N=400, K=8, alpha 1.5, beta 0.5)
    M = N = 400
    K = 8
    check_case(ctx, 0, ta, tb, M, N, K, 1.5, 0.5, lda=(K if ta else M), ldb=(N if tb else K), ldc=M)


@pytest.mark.parametrize("mn", [(150, 70), (398, 390)])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_vec_ragged_m(ctx, mn, ta, tb):
    # tests/sgemm/src/test.sgemm.js:239-296: k=13, ld rounded up to a multiple of 4
    M, N = mn
    K = 13
    up4 = lambda v: (v + 3) // 4 * 4
    check_case(ctx, 0, ta, tb, M, N, K, 1.5, 0.5, lda=up4(K if ta else M), ldb=up4(N if tb else K),
               ldc=M, seeds=(111, 112, 113))


def test_k0_is_beta_c_bit_exact(ctx):
    # tests/sgemm/src/test.sgemm.js:304-351
    C = orc.random_f32(16, -5, 5, 300)
    got = run_gemm(ctx, 0, 0, 1, 4, 4, 0, 1.5, np.zeros(3, np.float32), 4,
                   np.zeros(3, np.float32), 4, 0.5, C, 4)
    assert bits_equal(got, (np.float32(0.5) * C).astype(np.float32))
    for uplo in (1, 2):
        got = run_gemm(ctx, uplo, 0, 1, 4, 4, 0, 1.5, np.zeros(3, np.float32), 4,
                       np.zeros(3, np.float32), 4, 0.5, C, 4)
        keep = untouched_mask(4, 4, 4, 4, uplo)
        want = np.where(keep, C, (np.float32(0.5) * C).astype(np.float32))
        assert bits_equal(got, want)


@pytest.mark.parametrize("n", [7, 400])
@pytest.mark.parametrize("beta", [0.0, 0.5])
@pytest.mark.parametrize("uplo", [0, 1, 2])
def test_alpha_zero_reads_neither_a_nor_b(ctx, n, beta, uplo):
    # tests/sgemm/src/test.sgemm.js:399-443 (column-major indices here)
    A = orc.random_f32(n * n, -1, 1, 1)
    B = orc.random_f32(n * n, -1, 1, 2)
    C = orc.random_f32(n * n, -1, 1, 3)
    A[1 + 2 * n] = np.nan
    A[3] = -np.inf
    B[2 + 3 * n] = np.inf
    if beta == 0:
        C[4 + 4 * n] = np.nan
    got = run_gemm(ctx, uplo, 0, 0, n, n, n, 0.0, A, n, B, n, beta, C, n)
    inside = ~untouched_mask(n, n, n, n, uplo)
    want = C.copy()
    want[inside] = (np.float32(beta) * C[inside]).astype(np.float32) if beta else 0.0
    assert bits_equal(got, want)


def test_beta_zero_ignores_nan_in_c(ctx):
    n = 150
    C = orc.random_f32(n * n, -1, 1, 3)
    C[0], C[5] = np.nan, np.inf
    A = orc.random_f32(n * n, -1, 1, 1)
    B = orc.random_f32(n * n, -1, 1, 2)
    got = run_gemm(ctx, 0, 0, 0, n, n, n, 1.5, A, n, B, n, 0.0, C, n)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("variant", ["ldc_pad4", "c_misaligned", "beta0_nan"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", [(1024, 768, 96), (2048, 4608, 40)])  # 64 / 128 tier (576 tiles)
def test_epilogue_paths(ctx, variant, ta, dtype, shape):
    """C one element off 16-byte alignment against aligned C: fp32 stores
    whole vectors of rows either way (dword-aligned 16-byte stores), fp64
    falls back to element-wise stores; ld padding kept bit-identical and
    beta == 0 never reading C."""
    m, n, k = shape
    ldc = m + 4
    gen = orc.random_f64 if dtype == np.float64 else orc.random_f32
    lda = k if ta else m
    A = gen(lda * (m if ta else k), -1, 1, 41)
    B = gen(k * n, -1, 1, 42)
    C = gen(ldc * n, -1, 1, 43)
    beta = 0.5
    if variant == "beta0_nan":
        C[::7] = np.nan
        beta = 0.0
    shift = 1 if variant == "c_misaligned" else 0
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC = ctx.upload(np.concatenate([np.zeros(shift, dtype), C]))
    call = ctx.dgemm if dtype == np.float64 else ctx.sgemm
    call(ta, 0, m, n, k, 1.25, dA, lda, dB, k, beta, dC.offset(shift), ldc)
    got = dC.to_host()[shift:]
    for d in (dA, dB, dC):
        d.free()
    C0 = np.where(np.isnan(C), 0.0, C).astype(np.float64) if beta == 0.0 else C.astype(np.float64)
    ref, absdot = orc.gemm_ld(0, ta, 0, m, n, k, 1.25, A.astype(np.float64), lda,
                              B.astype(np.float64), k, beta, C0, ldc)
    fac = gemm_forward_factor(got, ref, absdot, C0, m, n, k, 1.25, beta, ldc, 0,
                              dd=dtype == np.float64)
    assert fac <= 1.0, f"forward factor {fac}"
    keep = untouched_mask(m, n, ldc, n, 0)
    assert bits_equal(got[keep], C[keep]), "ld padding of C changed"


@pytest.mark.parametrize("mn", [(100, 100), (150, 70), (70, 150)])
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_sgemmtr_non_square_and_untouched_triangle(ctx, mn, uplo, ta, tb):
    # tests/sgemmtr/src/test.sgemmtr.js:253-323 (K=9, seeds 51/52/53)
    M, N = mn
    K = 9
    check_case(ctx, uplo, ta, tb, M, N, K, 1.5, 0.5, lda=(K if ta else M), ldb=(N if tb else K),
               ldc=M, seeds=(51, 52, 53))


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("nk", [(100, 37), (301, 64), (2048, 40)])
def test_ssyrk_multi_tile(ctx, uplo, trans, nk):
    n, k = nk
    check_case(ctx, uplo, trans, 0, n, n, k, 1.25, 0.75, lda=(k if trans else n), ldb=0, ldc=n + 3,
               syrk=True)


# --------------------------------------------------------- tiers, edges, ld
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("shape", [(2048, 2048, 40), (2047, 2049, 37), (2304, 2176, 65)])
def test_large_tier_shapes(ctx, ta, tb, shape):
    m, n, k = shape
    check_case(ctx, 0, ta, tb, m, n, k, 1.5, 0.5, lda=(k if ta else m), ldb=(n if tb else k), ldc=m)


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_odd_leading_dimensions(ctx, ta, tb):
    # ld = 1 (mod 64): every column start is misaligned (element-wise loads)
    m, n, k = 191, 193, 97
    ld = lambda r: ((r + 63) // 64) * 64 + 1
    check_case(ctx, 0, ta, tb, m, n, k, -0.75, 1.0, lda=ld(k if ta else m), ldb=ld(n if tb else k),
               ldc=ld(m))


def _restride(x, rows, cols, ld_from, ld_to):
    """Column-major rows x cols from leading dimension ld_from to ld_to (new
    gap cells NaN: they must never be read)."""
    out = np.full(ld_to * cols, np.nan, x.dtype)
    out.reshape(cols, ld_to)[:, :rows] = x.reshape(cols, ld_from)[:, :rows]
    return out


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("shape", [(1100, 1000, 700), (4100, 4100, 1100)])
def test_element_aligned_operands_bit_equal_to_aligned(ctx, ta, tb, shape):
    """fp32 operands that are only element-aligned (ld = 1 mod 64, and a base
    one float past a 16-byte boundary) take the LDS copies too (the register
    path for NN); the MFMA sequence does not depend on how a k-tile reaches
    LDS, so C must equal, bit for bit, the product of the same values stored
    16-byte aligned (ld a multiple of 64). The shapes put the launch on the
    64-tile tier and on the 128-tile tier with a split-k tail (1089 tiles:
    two rounds and 65 tail tiles in k-slices); both include edge tiles and
    a partial k-tile."""
    m, n, k = shape
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    up = lambda r: (r + 63) // 64 * 64
    odd = lambda r: up(r) + 1
    A = orc.random_f32(up(a_rows) * a_cols, -1, 1, 71)
    B = orc.random_f32(up(b_rows) * b_cols, -1, 1, 72)
    C = orc.random_f32(up(m) * n, -1, 1, 73)
    outs = []
    for form in ("aligned", "odd_ld", "odd_base"):
        if form == "aligned":
            lda, ldb, ldc, shift = up(a_rows), up(b_rows), up(m), 0
        else:
            lda, ldb, ldc, shift = odd(a_rows), odd(b_rows), odd(m), (1 if form == "odd_base" else 0)
            if form == "odd_base":
                lda, ldb = up(a_rows) + 4, up(b_rows) + 4  # ld a multiple of 4, base misaligned
        hA = _restride(A, a_rows, a_cols, up(a_rows), lda)
        hB = _restride(B, b_rows, b_cols, up(b_rows), ldb)
        hC = _restride(C, m, n, up(m), ldc)
        pad = lambda h: np.concatenate([np.zeros(shift, np.float32), h])
        dA, dB, dC = ctx.upload(pad(hA)), ctx.upload(pad(hB)), ctx.upload(hC)
        try:
            print(f"element-aligned case {form} ta={ta} tb={tb} {m}x{n}x{k}", flush=True)
            ctx.sgemm(ta, tb, m, n, k, 1.5, dA.offset(shift), lda, dB.offset(shift), ldb, 0.5, dC, ldc)
            got = dC.to_host()
        finally:
            for d in (dA, dB, dC):
                d.free()
        keep = np.ones((n, ldc), bool)
        keep[:, :m] = False
        assert bits_equal(got.reshape(n, ldc)[keep], hC.reshape(n, ldc)[keep]), f"{form}: C padding changed"
        outs.append(got.reshape(n, ldc)[:, :m])
    assert bits_equal(outs[1], outs[0]), "ld = 1 mod 64 differs from the aligned product"
    assert bits_equal(outs[2], outs[0]), "misaligned base differs from the aligned product"
    # and the product itself against the oracle on sampled columns
    cols = np.unique(np.linspace(0, n - 1, 9).astype(int))
    opA = (A.reshape(a_cols, up(a_rows))[:, :a_rows].T if not ta
           else A.reshape(a_cols, up(a_rows))[:, :a_rows]).astype(np.float64)
    opB = (B.reshape(b_cols, up(b_rows))[:, :b_rows].T if not tb
           else B.reshape(b_cols, up(b_rows))[:, :b_rows]).astype(np.float64)
    c0 = C.reshape(n, up(m))[cols, :m].T.astype(np.float64)
    ref = 1.5 * (opA @ opB[:, cols]) + 0.5 * c0
    bound = EPS32 * ((k + 1) * 1.5 * (np.abs(opA) @ np.abs(opB[:, cols])) + 0.5 * np.abs(c0))
    assert np.all(np.abs(outs[0][cols].T.astype(np.float64) - ref) <= bound)


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("shape", [(512, 512, 512), (700, 300, 1024), (33, 65, 17), (704, 704, 1000),
                                   (31, 1, 5)])
def test_small_kernel_shapes(ctx, ta, tb, shape):
    # one-launch path (32x32 tiles, k split across the block's waves): taken
    # while 64-tiles would fill under half the chip and k <= 1024; ragged
    # m / n / k and padded leading dimensions
    m, n, k = shape
    check_case(ctx, 0, ta, tb, m, n, k, 1.5, 0.5, lda=(k if ta else m) + 3, ldb=(n if tb else k) + 1,
               ldc=m + 2)


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("case", [((4096, 4096, 64), "aligned"), ((4000, 4036, 70), "aligned"),
                                  ((4000, 4036, 70), "ldc_odd"), ((4000, 4036, 70), "beta0")])
def test_large_aligned_tier(ctx, ta, case):
    # large aligned problems on the 128 tier (several full rounds, the LDS
    # copy loop): interior and ragged tiles in m, n and k, the element-wise
    # epilogue (ldc odd) and beta = 0
    (m, n, k), variant = case
    ldc = m + 1 if variant == "ldc_odd" else m
    beta = 0.0 if variant == "beta0" else 0.5
    check_case(ctx, 0, ta, 0, m, n, k, 1.25, beta, lda=(k if ta else m), ldb=k, ldc=ldc)


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("lda", [(1 << 21) - 4, (1 << 21) + 4])
def test_huge_leading_dimension(ctx, ta, lda):
    # Aligned operands are copied into LDS with 32-bit lane offsets from the
    # tile origin while 256 * ld * sizeof(T) stays below 2^31; a larger ld
    # (here 2^21 + 4 floats) runs the register-staged loads instead. Both
    # sides of that limit, for k-contiguous (ta = 1) and m-contiguous A.
    m, n, k = 130, 72, 48
    check_case(ctx, 0, ta, 0, m, n, k, 1.25, 0.5, lda=lda, ldb=k, ldc=m)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("shape", [(2048, 2048, 40), (2100, 1900, 33)])
def test_sgemmtr_large_tier(ctx, uplo, shape):
    m, n, k = shape
    check_case(ctx, uplo, 0, 1, m, n, k, 1.0, 0.25, lda=m, ldb=n, ldc=m + 1)


def test_small_sizes_sweep(ctx):
    rng = np.random.default_rng(0)
    for _ in range(60):
        m, n, k = (int(v) for v in rng.integers(1, 40, size=3))
        ta, tb, uplo = int(rng.integers(0, 2)), int(rng.integers(0, 2)), int(rng.integers(0, 3))
        lda = (k if ta else m) + int(rng.integers(0, 3))
        ldb = (n if tb else k) + int(rng.integers(0, 3))
        ldc = m + int(rng.integers(0, 3))
        alpha = float(rng.choice([1.0, -1.0, 0.5, 2.5]))
        beta = float(rng.choice([0.0, 1.0, -0.5]))
        check_case(ctx, uplo, ta, tb, m, n, k, alpha, beta, lda, ldb, ldc,
                   seeds=tuple(int(s) for s in rng.integers(0, 1 << 30, size=3)))


# ------------------------------------------------------------------- dgemm
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("shape", [(150, 150, 150), (400, 333, 129), (2048, 2048, 33)])
def test_dgemm_shapes(ctx, ta, tb, shape):
    m, n, k = shape
    check_case(ctx, 0, ta, tb, m, n, k, 1.0, 1.0, lda=(k if ta else m) + 1,
               ldb=(n if tb else k), ldc=m, dtype=np.float64, seeds=(3, 4, 5))


def test_dgemm_quick_return_and_padding(ctx):
    # tests/dgemm/src/test.dgemm.js:353-408: alpha=0 or k=0 with beta=1 leaves C
    # untouched; ld padding of C comes back bit-identical.
    n = 6
    C = orc.random_f64(n * n, -1, 1, 1030) * np.pi
    for alpha, k in ((0.0, n), (1.5, 0)):
        got = run_gemm(ctx, 0, 0, 0, n, n, k, alpha, orc.random_f64(n * max(k, 1), -1, 1, 1),
                       n, orc.random_f64(max(k, 1) * n, -1, 1, 2), max(k, 1), 1.0, C, n,
                       np.float64)
        assert bits_equal(got, C)
    check_case(ctx, 0, 0, 0, 4, n, 2, 1.5, 0.5, lda=4, ldb=2, ldc=n + 3, dtype=np.float64)


def test_dgemm_ieee_specials(ctx):
    # tests/dgemm/src/test.dgemm.js:410-452: Inf/NaN reach C as in real f64
    for n in (7, 150):
        A = orc.random_f64(n * n, -1, 1, 1)
        B = orc.random_f64(n * n, -1, 1, 2)
        C = orc.random_f64(n * n, -1, 1, 3)
        A[2 + 1 * n] = np.inf
        B[4 + 3 * n] = np.nan
        C[0], C[5] = np.nan, np.inf
        got = run_gemm(ctx, 0, 0, 0, n, n, n, 1.5, A, n, B, n, 0.0, C, n, np.float64)
        ref, _ = orc.gemm_ld(0, 0, 0, n, n, n, 1.5, A, n, B, n, 0.0, np.zeros(n * n), n)
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        fin = np.isfinite(ref)
        assert np.array_equal(got[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
        assert np.allclose(got[fin], ref[fin], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape,ta,tb", [((512, 512, 512), 0, 0), ((1024, 1100, 300), 1, 0),
                                         ((1024, 1100, 300), 0, 1), ((4096, 4096, 64), 1, 0)])
def test_sgemm_ieee_specials_every_tier(ctx, shape, ta, tb):
    # NaN / Inf planted in A and B reach C as in real arithmetic on every
    # path (one-launch small kernel, the 128 tier's LDS copies, the wide
    # tier): the NaN / Inf pattern of C equals the long-double oracle's
    m, n, k = shape
    lda, ldb = (k if ta else m), (n if tb else k)
    A = orc.random_f32(lda * (m if ta else k), -1, 1, 21)
    B = orc.random_f32(ldb * (k if tb else n), -1, 1, 22)
    C = orc.random_f32(m * n, -1, 1, 23)
    at_a = lambda i, kk: (kk + i * lda) if ta else (i + kk * lda)   # op(A)(i, kk)
    at_b = lambda kk, j: (j + kk * ldb) if tb else (kk + j * ldb)   # op(B)(kk, j)
    A[at_a(m // 3, k // 2)] = np.nan
    A[at_a(m - 1, 1)] = -np.inf
    B[at_b(k - 1, n // 5)] = np.inf
    got = run_gemm(ctx, 0, ta, tb, m, n, k, 1.5, A, lda, B, ldb, 0.5, C, m)
    ref, _ = orc.gemm_ld(0, ta, tb, m, n, k, 1.5, A.astype(np.float64), lda, B.astype(np.float64),
                         ldb, 0.5, C.astype(np.float64), m)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))
    inf = np.isinf(ref)
    assert np.array_equal(np.sign(got[inf]), np.sign(ref[inf]))
    assert np.isnan(got).any() and inf.any()
