"""CPU model of the small-GEMM kernel (wgblas_amd/csrc/gemm.hip,
small_operands / gemm_small_kernel, 16 waves splitting k).

Restates, per lane, which element of op(A) and op(B) each MFMA operand
register is loaded from (with the row and k clamps of partial tiles), plays
the fp32 16x16x4 MFMA's operand and accumulator layout over those values,
scatters the accumulators through out_row / out_col as the kernel's LDS
reduction does, and checks:
  * every element read lies inside the operand (rows < rows, k < K);
  * the 32x32 tile holds exactly op(A) op(B) on its in-range rows and
    columns (so k past K contributes zero and the row placement of the
    loaders matches the epilogue's);
for both operand layouts, ragged m / n / k and the first and last tiles.
"""
import itertools

import numpy as np
import pytest

TILE = 32
WAVES = 16


def load_operands(KC, X, rows, r0, K, k0, whole):
    """out[s][b] per lane (64 lanes) and the (row, k) each value came from.
    X(i, k) is op(X); reads outside rows x K raise."""
    out = np.zeros((64, 4, 2))
    for lane in range(64):
        g, i16 = lane >> 4, lane & 15
        if KC:
            kk = k0 + 4 * g
            for b in range(2):
                row = r0 + 16 * b + i16
                if not whole:
                    row = min(row, rows - 1)
                nv = K - kk
                kb = kk if kk < K else K - 1
                for c in range(4):
                    if whole:
                        k = kk + c
                        val = X[row, k] if (row < rows and k < K) else None
                        assert val is not None, "WHOLE read outside the operand"
                    else:
                        k = kb + (c if c < nv else 0)
                        assert 0 <= row < rows and 0 <= k < K, (row, k)
                        val = X[row, k] if c < nv else 0.0
                    out[lane, c, b] = val
        else:
            row = r0 + 2 * i16
            for s in range(4):
                kk = k0 + 4 * g + s
                if whole:
                    assert row + 1 < rows and kk < K, "WHOLE read outside the operand"
                    v = (X[row, kk], X[row + 1, kk])
                else:
                    kc = min(kk, K - 1)
                    ra, rb = min(row, rows - 1), min(row + 1, rows - 1)
                    assert 0 <= kc < K and 0 <= ra < rows and 0 <= rb < rows
                    v = (X[ra, kc], X[rb, kc]) if kk < K else (0.0, 0.0)
                out[lane, s, 0], out[lane, s, 1] = v
    return out


def out_row(AKC, i, q, lane):
    r = 4 * (lane >> 4) + q
    return 16 * i + r if AKC else 2 * r + i


def out_col(BKC, j, lane):
    i16 = lane & 15
    return 16 * j + i16 if BKC else 2 * i16 + j


def tile_product(AKC, BKC, A, B, m, n, K, tm, tn):
    """The kernel's 32x32 tile (tm, tn), all waves summed."""
    m0, n0 = tm * TILE, tn * TILE
    inside = m0 + TILE <= m and n0 + TILE <= n
    nch, nwhole = (K + 15) // 16, K // 16
    cpw = 1 if nch <= WAVES else 2 if nch <= 2 * WAVES else 4
    tile = np.zeros((TILE, TILE))
    # wave w loads chunks w + 16 i, i < cpw (those past k read zeros); the
    # sum over waves is order-free here
    for c in range(WAVES * cpw):
        whole = inside and c < nwhole
        a = load_operands(AKC, A, m, m0, K, 16 * c, whole)
        b = load_operands(BKC, B, n, n0, K, 16 * c, whole)
        acc = np.zeros((2, 2, 64, 4))  # [i][j][lane][q]
        for s in range(4):
            for i in range(2):
                for j in range(2):
                    # MFMA 16x16x4: A_blk[r][kk] from lane r + 16 kk, B_blk[kk][c]
                    # from lane c + 16 kk; lane c + 16 g register q holds C[4g+q][c]
                    Ab = np.array([[a[r + 16 * kk, s, i] for kk in range(4)] for r in range(16)])
                    Bb = np.array([[b[cc + 16 * kk, s, j] for cc in range(16)] for kk in range(4)])
                    Cb = Ab @ Bb
                    for lane in range(64):
                        g, cc = lane >> 4, lane & 15
                        for q in range(4):
                            acc[i, j, lane, q] += Cb[4 * g + q, cc]
        for i, j, lane, q in itertools.product(range(2), range(2), range(64), range(4)):
            tile[out_row(AKC, i, q, lane), out_col(BKC, j, lane)] += acc[i, j, lane, q]
    return tile


CASES = [
    # (m, n, K, tiles to check)
    (64, 64, 32, [(0, 0), (1, 1)]),
    (33, 47, 19, [(0, 0), (1, 1), (1, 0)]),
    (5, 3, 1, [(0, 0)]),
    (40, 70, 45, [(1, 2), (0, 2)]),
    (32, 32, 300, [(0, 0)]),     # two chunks per wave, the last ones partly past k
    (20, 36, 1000, [(0, 1)]),    # four chunks per wave
]


@pytest.mark.parametrize("AKC,BKC", list(itertools.product([False, True], [False, True])))
@pytest.mark.parametrize("m,n,K,tiles", CASES)
def test_small_kernel_model(AKC, BKC, m, n, K, tiles):
    rng = np.random.default_rng(m * 1000 + n * 10 + K)
    A = rng.standard_normal((m, K))   # op(A): m x K
    B = rng.standard_normal((n, K))   # op(B)^T: n x K, so op(B)(k, j) = B[j, k]
    want = A @ B.T
    for tm, tn in tiles:
        got = tile_product(AKC, BKC, A, B, m, n, K, tm, tn)
        r, c = min(TILE, m - tm * TILE), min(TILE, n - tn * TILE)
        ref = want[tm * TILE:tm * TILE + r, tn * TILE:tn * TILE + c]
        assert np.allclose(got[:r, :c], ref, rtol=1e-12, atol=1e-12), (tm, tn)


def test_planted_row_swap_is_caught():
    # the model must see a wrong placement: swap the mn-contiguous virtual
    # blocks in out_col and the product no longer matches
    global out_col
    saved = out_col
    try:
        out_col = lambda BKC, j, lane: (16 * j + (lane & 15)) if BKC else 2 * (lane & 15) + (1 - j)
        rng = np.random.default_rng(7)
        A, B = rng.standard_normal((32, 16)), rng.standard_normal((32, 16))
        got = tile_product(False, False, A, B, 32, 32, 16, 0, 0)
        assert not np.allclose(got, A @ B.T)
    finally:
        out_col = saved
