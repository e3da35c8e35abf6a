"""CPU: every load window of the whole-wave GEMV lanes stays inside the weight
buffer, for every row shape the lanes accept.

The whole-wave GEMV (aero_amd/csrc/gemv.hip, Lane64<TYPE>::load, used by
gemv64_kernel and gemv64_fused_kernel) gives lane l of step st the block
kc = min(st*16 + l/4, n_blk-1) (Q8_0: the block pair kc = min(st*128 + 2l,
n_blk-2)) of row min(row, n_rows-1) and loads 16-byte pieces from there. A
matrix is admitted when its base is 16-byte aligned and its rows are whole 16
bytes, or, for Q8_0 only, whole 8 bytes with the buffer padded to the next
16-byte boundary after the last row (lanes64_ok, gemv.hip:1612-1618). Q8_0
rows 8 bytes past a boundary (952-byte rows of 896 values, 680 of 640) read
five 16-byte pieces from the boundary at or below their blocks.

The addresses are restated here with Python integers, the kernel's formulas
piece by piece, and each window is checked against [w, w + w_bytes). The old
Q8_0 base, rowp + (ob - ph) formed in 32-bit arithmetic, wrapped to ~4 GiB
past the row on rows that start 8 bytes past a boundary (a GPU memory fault
at the first 896-column parity case); it is kept as a planted mistake that
this check must catch.
"""
import numpy as np
import pytest

from aero_amd import workloads as W

STEP_COLS = 4096          # kStepCols: 64 lanes x 64 columns
BASE = 0x7F3A_0000_0000   # any 16-byte aligned address


def lanes64_ok(dtype, rb, n_rows, w_bytes):
    if rb % 16 == 0:
        return True
    if dtype != W.Q8_0 or rb % 8 != 0 or n_rows <= 0:
        return False
    end = n_rows * rb
    return w_bytes >= end + ((16 - (end & 15)) & 15)


def windows(dtype, rowp, n_cols, old_q8=False):
    """(first byte, one past the last byte) of every 16/8/2-byte load of every
    lane and step of one row starting at rowp: arrays of Python-int-valued
    int64 (addresses stay below 2**63)."""
    bv, bb = W.BLOCK[dtype]
    n_blk = n_cols // bv
    n_st = -(-n_cols // STEP_COLS)
    st = np.arange(n_st, dtype=np.int64)[:, None]
    l = np.arange(64, dtype=np.int64)[None, :]
    spans = []
    if dtype == W.Q8_0:
        kc = np.minimum(st * 128 + 2 * l, n_blk - 2)
        ob = kc * 34
        a = rowp + ob
        ph = a & 15
        if old_q8:
            base = rowp + ((ob - ph) & 0xFFFFFFFF)
        else:
            base = a - ph
        assert np.all((base + ph == a) | old_q8)
        spans.append((base, base + 80))
        return spans
    kc = np.minimum(st * 16 + (l >> 2), n_blk - 1)
    j = l & 3
    ob = kc * bb
    if dtype == W.Q4_K:
        oq = ob + 16 + 32 * j
        spans += [(rowp + ob, rowp + ob + 16), (rowp + oq, rowp + oq + 32)]
    elif dtype == W.Q5_K:
        oq = ob + 48 + 32 * j
        spans += [(rowp + ob, rowp + ob + 48), (rowp + oq, rowp + oq + 32)]
    elif dtype == W.IQ4_XS:
        oq = ob + 8 + 32 * j
        spans += [(rowp + ob, rowp + ob + 8), (rowp + oq, rowp + oq + 32)]
    elif dtype == W.Q6_K:
        ph = ob & 15
        bl = rowp + (ob - ph)
        h, a = j >> 1, j & 1
        spans += [(bl + 64 * h + 32 * a, bl + 64 * h + 32 * a + 48),
                  (bl + 128 + 32 * h, bl + 128 + 32 * h + 48),
                  (rowp + ob + 192 + 8 * h + 2 * a, rowp + ob + 192 + 8 * h + 2 * a + 6),
                  (rowp + ob + 208, rowp + ob + 210)]
    else:
        raise ValueError(dtype)
    return spans


def check_matrix(dtype, n_rows, n_cols, old_q8=False):
    """Number of windows outside [BASE, BASE + w_bytes) with the smallest
    w_bytes lanes64_ok admits, over every row; None when not admitted."""
    bv, bb = W.BLOCK[dtype]
    rb = (n_cols // bv) * bb
    end = n_rows * rb
    w_bytes = end + (((16 - (end & 15)) & 15) if rb % 16 else 0)
    if not lanes64_ok(dtype, rb, n_rows, w_bytes):
        return None
    bad = 0
    rows = np.arange(n_rows, dtype=np.int64)
    # a row's windows depend on its start modulo 16 and on whether it is the
    # last row; every row is checked all the same
    for row in rows:
        rowp = BASE + int(row) * rb
        for lo, hi in windows(dtype, rowp, n_cols, old_q8):
            bad += int(np.count_nonzero((lo < BASE) | (hi > BASE + w_bytes)))
    return bad


Q8_COLS = [128, 256, 640, 896, 1152, 2048, 2176, 4096, 4864, 5120, 8192, 8320]
Q8_ROWS = [1, 2, 3, 7, 64, 129]


@pytest.mark.parametrize("n_cols", Q8_COLS)
def test_q8_0_windows_inside_buffer(n_cols):
    for n_rows in Q8_ROWS:
        bad = check_matrix(W.Q8_0, n_rows, n_cols)
        if bad is None:
            continue
        assert bad == 0, (n_rows, n_cols)


def test_q8_0_eight_byte_rows_are_admitted_and_checked():
    """952- and 680-byte rows (896 and 640 values) are admitted with padding
    and every window stays inside."""
    for n_cols in (896, 640):
        rb = n_cols // 32 * 34
        assert rb % 16 == 8
        for n_rows in (1, 2, 3, 896, 4864 // 8):
            assert check_matrix(W.Q8_0, n_rows, n_cols) == 0, (n_rows, n_cols)


def test_planted_32bit_base_is_caught():
    """The old base rowp + (ob - ph) in 32-bit arithmetic wraps on rows that
    start 8 bytes past a 16-byte boundary: the check must see it."""
    assert check_matrix(W.Q8_0, 2, 896, old_q8=True) > 0
    assert check_matrix(W.Q8_0, 3, 640, old_q8=True) > 0
    # on 16-byte rows ph never exceeds ob, so the old formula was safe there
    assert check_matrix(W.Q8_0, 3, 4096, old_q8=True) == 0


@pytest.mark.parametrize("dtype", [W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS])
def test_k_quant_windows_inside_buffer(dtype):
    admitted = 0
    for n_cols in (256, 512, 768, 1024, 2048, 2304, 4096, 4352, 5120, 8192, 14336):
        for n_rows in (1, 2, 3, 17):
            bad = check_matrix(dtype, n_rows, n_cols)
            if bad is None:
                continue
            admitted += 1
            assert bad == 0, (dtype, n_rows, n_cols)
    assert admitted > 0


def test_rows_not_admitted():
    """Rows of neither whole 16 bytes nor (Q8_0) whole 8 bytes stay on the
    word GEMV: Q8_0 of 32 values (34 bytes), Q6_K of 256 (210 bytes)."""
    assert check_matrix(W.Q8_0, 4, 32) is None
    assert check_matrix(W.Q6_K, 4, 256) is None
    # Q8_0 8-byte rows without the padding after the last row
    rb = 896 // 32 * 34
    assert not lanes64_ok(W.Q8_0, rb, 3, 3 * rb)
