"""GPU parity of the wide fp32 GEMM tier (256 x 128 tiles of C, two blocks of
four waves per CU, accumulators in AGPRs, k-tiles of 16 floats in a ring of
three LDS stages).

sgemm takes that tier for 16-byte aligned operands and C, m % 256 == 0,
n % 128 == 0, k a multiple of 16 with k >= 1024, when its tiles fill whole
rounds of two blocks per CU (a multiple of 512 tiles on MI355X). The cases
below qualify (one round each), with k giving 64, 65 and 66 k-tiles (an odd
count takes the last k-tile after the two-k-tile loop; the copies past the
last k-tile re-read it into a stage nobody reads). The same product with
ldc = m + 1 (C not vector-accessible) runs on the 128 x 128 tier; both
tiers add the same MFMA products in the same k order, so the two results
must be equal bit for bit. The wide result is also checked against float64
under the reference's forward-error bound (sampled rows and columns plus a
Freivalds projection over all of C).
"""
import numpy as np
import pytest

from tests.helpers import bits_equal, check_gemm_props, cm_view, op

pytestmark = pytest.mark.gpu


def _pair(ctx, ta, tb, m, n, k, alpha, beta, seed, nan_c=False):
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb = a_rows, b_rows
    sa, sb = lda * a_cols, ldb * b_cols
    sc1, sc2 = m * n, (m + 1) * n
    buf = ctx.empty(sa + sb + sc1 + sc2, np.float32)
    ctx.fill_uniform(buf, -1.0, 1.0, seed)
    host = buf.to_host()
    C0 = cm_view(host[sa + sb:sa + sb + sc1], m, n, m).copy()
    c = host.copy()
    if nan_c:
        # beta = 0 must not read C: NaN there may not reach the result
        c[sa + sb:] = np.nan
    else:
        # both C's start from the same values
        cm_view(c[sa + sb + sc1:], m, n, m + 1)[:, :] = C0
    ctx.h2d(buf.ptr, c)
    pa, pb = buf.offset(0), buf.offset(sa)
    ctx.sgemm(ta, tb, m, n, k, alpha, pa, lda, pb, ldb, beta, buf.offset(sa + sb), m)
    ctx.sgemm(ta, tb, m, n, k, alpha, pa, lda, pb, ldb, beta, buf.offset(sa + sb + sc1), m + 1)
    out = buf.to_host()
    buf.free()
    wide = cm_view(out[sa + sb:sa + sb + sc1], m, n, m)
    tier128 = cm_view(out[sa + sb + sc1:], m, n, m + 1)
    A = op(cm_view(host[:sa], a_rows, a_cols, lda), ta)
    B = op(cm_view(host[sa:sa + sb], b_rows, b_cols, ldb), tb)
    return wide, tier128, A, B, C0


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(4096, 4096, 1040), (8192, 2048, 1024), (2048, 8192, 1056)])
def test_wide_tier_matches_128_tier(ctx, ta, tb, m, n, k):
    wide, tier128, A, B, C0 = _pair(ctx, ta, tb, m, n, k, 1.5, 0.5, seed=21 + 2 * ta + tb)
    assert bits_equal(wide, tier128), "wide tier differs from the 128 tier"
    edges = (127, 128, 255, 256, m - 256, m - 129, n - 128, n - 65)
    check_gemm_props(wide, C0, A, B, 1.5, 0.5, k, rows=tuple(r for r in edges if r < m),
                     cols=tuple(c for c in edges if c < n), seed=ta * 2 + tb)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_wide_tier_beta_zero_never_reads_c(ctx, ta, tb):
    wide, tier128, A, B, _ = _pair(ctx, ta, tb, 4096, 4096, 1024, -0.75, 0.0, seed=29, nan_c=True)
    assert np.all(np.isfinite(wide))
    assert bits_equal(wide, tier128)
    check_gemm_props(wide, np.zeros_like(wide), A, B, -0.75, 0.0, 1024, seed=5)
