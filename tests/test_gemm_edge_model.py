"""CPU model of the GEMM edge-tile loads (wgblas_amd/csrc/gemm.hip,
Stager::init / init_edge / load<false, true>).

Edge tiles stream whole k-tiles (all but the last whole one) without element
guards: a lane whose rows lie past rows_total reads at `fb` (row
rows_total-1), and a partly in-range mn-contiguous vector reads past its
column end. This restates those address computations and checks that every
element read lies inside the operand matrix for many shapes, leading
dimensions (down to 1), tile sizes, element types and split-k starting
tiles: a partly in-range vector overruns its column by at most VW-1 elements
and at least BK columns follow the last column read this way.

The fp32 LDS copies (Stager::init_copy / load_lds: 16-byte aligned operands,
and since they also take element-aligned ones, any ld) read the same
addresses except that a k-contiguous lane reads the 16-byte chunk the LDS
swizzle places at its slot, chunk kv ^ (row & 7) of its row instead of kv
(copy_shift); COPY adds that shift.
"""
import pytest

THREADS = 256


def max_read_offset(KC, BT, VW, BK, rows_total, K, ld, kt0, COPY=False):
    """Largest and smallest element offset read by EDGE loads, or None."""
    LOADS, VPK = BT // 32, BT // VW
    KROWS = THREADS // VPK
    nkt_whole = K // BK - kt0 - 1
    lo, hi = None, None
    tiles = (rows_total + BT - 1) // BT
    for tm in range(tiles):
        row0 = tm * BT
        for t in range(THREADS):
            if KC:
                row, kv = t // 8, t % 8
                row_first = row0 + row
                base = (row0 + row) * ld + kv * VW + kt0 * BK
                r_step, k_step = 32 * ld, BK
                valid = rows_total - row_first
                nvr = 0 if valid <= 0 else min((valid + 31) // 32, LOADS)
                fb = base + (rows_total - 1 - row_first) * (r_step // 32)
                shift = ((kv ^ (row & 7)) - kv) * VW if COPY else 0
            else:
                mv, kk = t % VPK, t // VPK
                row_first = row0 + mv * VW
                base = row0 + mv * VW + kk * ld + kt0 * BK * ld
                r_step, k_step = KROWS * ld, BK * ld
                vok = rows_total - row_first > 0
                fb = base + (rows_total - 1 - row_first)
            for kt in range(max(nkt_whole, 0)):
                for r in range(LOADS):
                    q = base + kt * k_step + r * r_step
                    if KC:
                        a = (q if r < nvr else fb + kt * k_step) + shift
                    else:
                        a = q if vok else fb + kt * k_step + r * r_step
                    lo = a if lo is None else min(lo, a)
                    hi = a + VW - 1 if hi is None else max(hi, a + VW - 1)
    return lo, hi


CASES = []
for KC in (True, False):
    for VW, BK in ((4, 32), (2, 16)):
        for BT in (64, 128):
            for rows_total in (1, 2, 3, 5, 63, 65, 127, 129, 191):
                for K in (3 * BK - 1, 4 * BK, 5 * BK + 3):
                    for pad in (0, 1, 64):
                        for kt0 in (0, 1):
                            for copy in ((False, True) if VW == 4 else (False,)):
                                CASES.append((KC, BT, VW, BK, rows_total, K, pad, kt0, copy))


@pytest.mark.parametrize("KC,BT,VW,BK,rows_total,K,pad,kt0,copy", CASES)
def test_edge_loads_stay_inside_the_matrix(KC, BT, VW, BK, rows_total, K, pad, kt0, copy):
    ld = (K if KC else rows_total) + pad
    lo, hi = max_read_offset(KC, BT, VW, BK, rows_total, K, ld, kt0, copy)
    if lo is None:
        return
    last = (rows_total - 1) * ld + K - 1 if KC else (K - 1) * ld + rows_total - 1
    assert lo >= 0 and hi <= last, (lo, hi, last)


def copy_chunk(t):
    """16-byte chunk of its row (0..7 in a 32-float k-tile) that thread t's
    fp32 LDS copy reads: chunk kv ^ (row & 7) (Stager::init, copy_shift)."""
    row, kv = t // 8, t % 8
    return (kv ^ (row & 7))


def test_copy_chunks_cover_each_row_k_tile_once():
    # The 8 lanes of a row copy its 8 chunks of the k-tile, each exactly
    # once, and never a chunk of another k-tile: so the copies' addresses are
    # the register path's, permuted inside each row's k-tile (which the
    # bounds above then cover), and every LDS slot gets its element.
    for row in range(THREADS // 8):
        chunks = sorted(copy_chunk(8 * row + kv) for kv in range(8))
        assert chunks == list(range(8)), (row, chunks)
