"""GPU parity: the split-x fp16 matrix-core GEMM (aero_hip_matmul with a
workspace, Q4_K / Q5_K / Q8_0 / Q6_K / IQ4_XS, 32 or more tokens) against the
oracle's restatement of the reference's matmul (src/kernels.cpp:337-458,520-538)
and against the exact product.

Tolerances: 1e-5 relative to the output's scale against the oracle (the
reference's RTOL for fp32 ops, tests/test_transformer_native.py:34-37). Each
token's x is scaled by a power of two per super-block and split into two fp16
parts, so every value keeps 22 significant bits (relative error <= 2^-22);
the tests below also check extreme and mixed magnitudes, where the result must
equal the float64 product of the dequantised weights to ~1e-6 of the scale,
and the split's per-value bound on crafted values.
"""
import numpy as np
import pytest

from conftest import RTOL, rel_to_scale
from aero_amd import _lib, native, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

KTYPES = [W.Q4_K, W.Q5_K, W.Q8_0]


def table(t, n_rows, n_cols, rng):
    return W.make_table(t, n_rows * n_cols // W.BLOCK[t][0], rng)


def gpu_matmul(t, w, X, n_rows, split=True):
    X = np.ascontiguousarray(np.atleast_2d(X), np.float32)
    T, n_cols = X.shape
    y = DA.empty((T, n_rows))
    ops.matvec(t, DA.from_numpy(w), DA.from_numpy(X), y, n_rows, n_cols, T, split=split)
    return y.numpy()


def exact(oracle, t, w, X, n_rows):
    """float64 X @ W^T over the reference's dequantised weights."""
    n_cols = X.shape[1]
    Wd = oracle.dequant(t, w, n_rows * n_cols).reshape(n_rows, n_cols).astype(np.float64)
    return X.astype(np.float64) @ Wd.T


def test_workspace_sizes(hip):
    L = _lib.lib()
    for t in KTYPES:
        assert L.aero_hip_matmul_workspace(t, 4096, 512) >= 512 * 4096 * 4   # 2 fp16 parts
        assert L.aero_hip_matmul_workspace(t, 4096, 33) >= 64 * 4096 * 4  # padded to 32s
        assert L.aero_hip_matmul_workspace(t, 100, 64) == 0                # not whole blocks
    assert L.aero_hip_matmul_workspace(W.Q6_K, 4096, 512) >= 512 * 4096 * 4
    assert L.aero_hip_matmul_workspace(W.Q6_K, 5120, 512) == 0   # rows not 16-byte aligned
    assert L.aero_hip_matmul_workspace(W.IQ4_XS, 4096, 512) >= 512 * 4096 * 4
    assert L.aero_hip_matmul_workspace(W.IQ4_XS, 768, 512) == 0   # odd block count
    assert L.aero_hip_matmul_workspace(W.F32, 4096, 512) == 0


@pytest.mark.parametrize("t", KTYPES)
@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (100, 1024, 40), (130, 2048, 33), (257, 4096, 100), (64, 14336, 64), (1000, 256, 32),
    (129, 512, 95),
])
def test_split_gemm_vs_oracle(hip, oracle, t, n_rows, n_cols, n_tok):
    """Partial row tiles (rows not a multiple of 128), partial token tiles (33,
    40, 95, 100 tokens), one to 56 super-blocks a row."""
    rng = np.random.default_rng(n_rows * 31 + n_cols + n_tok + t)
    w = table(t, n_rows, n_cols, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"split gemm type={t} rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    assert rel_to_scale(got, gpu_matmul(t, w, X, n_rows, split=False)) <= RTOL


@pytest.mark.parametrize("t", KTYPES)
def test_split_gemm_magnitudes(hip, oracle, t):
    """Tokens at 1e-30 and 1e30 scale, an all-zero token, a token of one
    outlier among small values, fp32 subnormals and values equal to 2^-16 of
    their token's largest: all within 1e-6 of the exact product's scale (per
    token), the zero token exactly zero. The subnormal token's outputs are
    themselves subnormal (~13 significant bits): there each super-block's
    scaled-back sum is rounded once to the fp32 grid (2^-149) as it is added,
    so the bound gains one grid step a super-block."""
    rng = np.random.default_rng(5 + t)
    n_rows, n_cols = 96, 1024
    w = table(t, n_rows, n_cols, rng)
    base = rng.standard_normal((8, n_cols)).astype(np.float32)
    X = np.empty((40, n_cols), np.float32)
    X[:] = rng.standard_normal((40, n_cols)).astype(np.float32)
    X[0] = base[0] * np.float32(1e-30)
    X[1] = base[1] * np.float32(1e30)
    X[2] = 0.0
    X[3] = base[3] * np.float32(1e-3)
    X[3, 17] = 1e4                                      # outlier among small values
    X[4] = base[4] * np.float32(1e-41)                  # fp32 subnormals
    X[5] = np.float32(1.0)
    X[5, ::3] = np.float32(2.0 ** -16)                  # the exactness threshold
    got = gpu_matmul(t, w, X, n_rows).astype(np.float64)
    want = exact(oracle, t, w, X, n_rows)
    assert not got[2].any()
    for i in range(40):
        if i == 2:
            continue
        scale = np.abs(want[i]).max()
        assert np.abs(got[i] - want[i]).max() <= 1e-6 * scale + (n_cols // 256) * 2.0 ** -149, i


def test_split_gemm_per_value_bound(hip, oracle):
    """The split's bound, value by value: a one-hot weight row picks x[c]
    alone, so y[t, r] is the token's x[c] as the GEMM represents it (scaled
    by its super-block's power of two, split, scaled back). Values with 24
    significant bits come back within 2^-22 relative; values with 22 or
    fewer come back exactly; values far below their block's largest within
    2^-39 of that largest. The oracle restates no split: the bound checked
    is the arithmetic's own, on weights the oracle dequantises to one-hot
    rows."""
    t = W.Q4_K
    n_cols, n_rows, T = 512, 64, 32
    rng = np.random.default_rng(29)
    # rows 0..63 pick columns 8r: Q4_K with d = 1, dmin = 0, scales 1, one
    # quant of 1 at the picked column, zeros elsewhere
    w = np.zeros((n_rows, n_cols // 256, 144), np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[:, :, 4:8] = 1          # sc of sub-blocks 0-3 = 1 (low 6 bits), m = 0
    w[:, :, 12:16] = 0x01     # sc of sub-blocks 4-7 = 1
    cols = 8 * np.arange(n_rows)
    for r, c in enumerate(cols):
        sb, v = divmod(c, 256)
        j, rem = divmod(v, 64)
        hi, i = divmod(rem, 32)
        w[r, sb, 16 + 32 * j + i] |= (1 << (4 * hi))
    w = w.reshape(-1)
    Wd = oracle.dequant(t, w, n_rows * n_cols).reshape(n_rows, n_cols)
    assert np.array_equal(np.argmax(Wd, axis=1), cols) and Wd.sum() == n_rows
    X = (rng.standard_normal((T, n_cols)) * 3).astype(np.float32)
    X[1, cols] = np.float32(1.0) + np.float32(2.0 ** -20) * np.arange(n_rows)  # 21 bits
    X[2, :] = np.float32(1000.0)
    X[2, cols[::2]] = np.float32(1e-9)               # tiny beside their block's largest
    got = gpu_matmul(t, w, X, n_rows).astype(np.float64)
    want = X[:, cols].astype(np.float64)
    normal = np.ones(want.shape, bool)
    normal[2, ::2] = False
    rel = np.abs(got - want)[normal] / np.abs(want)[normal]
    assert rel.max() <= 2.0 ** -22, rel.max()
    assert np.array_equal(got[1], want[1])            # 22 or fewer bits: exact
    # the scaled block's largest is in [2^14, 2^15): 2^-25 absolute there
    assert np.abs(got[2, ::2] - want[2, ::2]).max() <= 1000.0 * 2.0 ** -39


def q8_blocks(q, d):
    """Q8_0 rows from int8 quants q [rows, cols] and fp16 scales d [rows, cols/32]."""
    rows, cols = q.shape
    blk = np.empty((rows, cols // 32, 34), np.uint8)
    blk[:, :, 0:2] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(
        rows, cols // 32, 2)
    blk[:, :, 2:] = q.astype(np.int8).view(np.uint8).reshape(rows, cols // 32, 32)
    return blk.reshape(-1)


def test_split_gemm_q8_identity(hip, oracle):
    """Q8_0 rows that pick one column each (d = 1, q = 1 there, 0 elsewhere),
    every column of 1024 once: y equals x value for value, for x of 22
    significant bits within 2^7 of their super-block's largest (the two fp16
    parts then hold them exactly). Each column
    position of the even and odd blocks of a pair comes from a different lane
    and dword of the weight rows, so a wrong operand order shows."""
    t, n = W.Q8_0, 1024
    rng = np.random.default_rng(41)
    perm = rng.permutation(n)
    q = np.zeros((n, n), np.int8)
    q[np.arange(n), perm] = 1
    w = q8_blocks(q, np.ones((n, n // 32), np.float32))
    Wd = oracle.dequant(t, w, n * n).reshape(n, n)
    assert np.array_equal(np.argmax(Wd, axis=1), perm) and Wd.sum() == n
    X = (rng.uniform(0.05, 4.0, (48, n)) * rng.choice([-1, 1], (48, n))).astype(np.float32)
    X = (X.view(np.uint32) & np.uint32(0xFFFFFFFC)).view(np.float32)   # 22 bits
    got = gpu_matmul(t, w, X, n)
    assert np.array_equal(got, X[:, perm])


def test_split_gemm_q8_full_range(hip, oracle):
    """Q8_0 with every int8 quant (-128 included), negative, subnormal and
    large fp16 scales, against the oracle and the exact product."""
    t, n_rows, n_cols, T = W.Q8_0, 160, 2048, 70
    rng = np.random.default_rng(43)
    q = rng.integers(-128, 128, size=(n_rows, n_cols)).astype(np.int8)
    q[0, :256] = -128
    q[1, :256] = 127
    d = (rng.standard_normal((n_rows, n_cols // 32)) * 0.01).astype(np.float32)
    d[2] = np.float32(3e-7)     # fp16 subnormals
    d[3] = np.float32(-60000.0)
    d[4, ::2] = 0.0
    w = q8_blocks(q, d)
    X = rng.standard_normal((T, n_cols)).astype(np.float32)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    want = exact(oracle, t, w, X, n_rows)
    for r in range(5):
        scale = np.abs(want[:, r]).max()
        assert np.abs(got[:, r] - want[:, r]).max() <= 1e-6 * scale, r


@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (100, 2048, 40), (257, 4096, 100), (64, 14336, 64), (130, 6144, 33),
])
def test_split_gemm_q6k_vs_oracle(hip, oracle, n_rows, n_cols, n_tok):
    """Q6_K rows of 8 or more blocks (16-byte aligned): blocks at odd indices
    start 2 bytes past a 4-byte boundary."""
    t = W.Q6_K
    rng = np.random.default_rng(n_rows + n_cols + n_tok)
    w = table(t, n_rows, n_cols, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"split gemm Q6_K rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    assert rel_to_scale(got, gpu_matmul(t, w, X, n_rows, split=False)) <= RTOL


def q6k_blocks(q, sc, d):
    """Q6_K rows from 6-bit quants q [rows, cols] (0..63), int8 scales sc
    [rows, cols/16] and fp16 d [rows, cols/256], in the layout of
    src/kernels.cpp:427-458."""
    rows, cols = q.shape
    nb = cols // 256
    blk = np.zeros((rows, nb, 210), np.uint8)
    v = np.arange(256)
    n, r = v // 128, v % 128
    Q, l = r // 32, r % 32
    qli = 64 * n + l + 32 * (Q & 1)
    qhi = 128 + 32 * n + l
    qb = q.reshape(rows, nb, 256).astype(np.uint8)
    for i in range(256):
        lo = qb[:, :, i] & 15
        blk[:, :, qli[i]] |= (lo << (4 * (Q[i] >> 1))).astype(np.uint8)
        blk[:, :, qhi[i]] |= ((qb[:, :, i] >> 4) << (2 * Q[i])).astype(np.uint8)
    blk[:, :, 192:208] = sc.astype(np.int8).view(np.uint8).reshape(rows, nb, 16)
    blk[:, :, 208:210] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(
        rows, nb, 2)
    return blk.reshape(-1)


def test_split_gemm_q6k_identity(hip, oracle):
    """Q6_K rows that pick one column each (d = 1, scales 1, q - 32 = 1
    there, 0 elsewhere), every column of 2048 once: y equals x value for
    value (x of 22 significant bits within 2^7 of their super-block's
    largest). Each quarter, lane group and block parity reads other words."""
    t, n = W.Q6_K, 2048
    rng = np.random.default_rng(47)
    perm = rng.permutation(n)
    q = np.full((n, n), 32, np.int64)
    q[np.arange(n), perm] = 33
    w = q6k_blocks(q, np.ones((n, n // 16)), np.ones((n, n // 256), np.float32))
    Wd = oracle.dequant(t, w, n * n).reshape(n, n)
    assert np.array_equal(np.argmax(Wd, axis=1), perm) and Wd.sum() == n
    X = (rng.uniform(0.05, 4.0, (40, n)) * rng.choice([-1, 1], (40, n))).astype(np.float32)
    X = (X.view(np.uint32) & np.uint32(0xFFFFFFFC)).view(np.float32)
    got = gpu_matmul(t, w, X, n)
    assert np.array_equal(got, X[:, perm])


def test_split_gemm_q6k_full_range(hip, oracle):
    """Q6_K with every 6-bit quant and scales -128..127 (sc*(q-32) up to
    4096, beyond fp16's exact integers), large, subnormal and negative d,
    against the oracle and the exact product."""
    t, n_rows, n_cols, T = W.Q6_K, 96, 4096, 48
    rng = np.random.default_rng(53)
    q = rng.integers(0, 64, size=(n_rows, n_cols))
    sc = rng.integers(-128, 128, size=(n_rows, n_cols // 16))
    q[0], sc[0] = 0, -128            # (q - 32) * sc = 4096
    q[1], sc[1] = 63, -127           # -3937: odd beyond 2048
    d = (rng.standard_normal((n_rows, n_cols // 256)) * 0.01).astype(np.float32)
    d[2] = np.float32(3e-7)
    d[3] = np.float32(-30000.0)
    w = q6k_blocks(q, sc, d)
    X = rng.standard_normal((T, n_cols)).astype(np.float32)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    want = exact(oracle, t, w, X, n_rows)
    for r in range(n_rows):
        scale = np.abs(want[:, r]).max()
        assert np.abs(got[:, r] - want[:, r]).max() <= 2e-6 * scale, r


@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (100, 512, 40), (257, 4096, 100), (64, 14336, 64), (130, 1536, 33),
])
def test_split_gemm_iq4xs_vs_oracle(hip, oracle, n_rows, n_cols, n_tok):
    """IQ4_XS rows of an even block count (16-byte aligned)."""
    t = W.IQ4_XS
    rng = np.random.default_rng(3 * n_rows + n_cols + n_tok)
    w = table(t, n_rows, n_cols, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"split gemm IQ4_XS rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    assert rel_to_scale(got, gpu_matmul(t, w, X, n_rows, split=False)) <= RTOL


def test_split_gemm_iq4xs_full_range(hip, oracle):
    """IQ4_XS with every codebook entry and every 6-bit scale (ls - 32 from
    -32 to 31, zero included), large, subnormal and negative d, against the
    oracle and the exact product; one row of codebook entry 8 (value 1)
    but for column 5 of each block (113)."""
    t, n_rows, n_cols, T = W.IQ4_XS, 96, 2048, 40
    rng = np.random.default_rng(59)
    blk = rng.integers(0, 256, size=(n_rows, n_cols // 256, 136), dtype=np.uint8)
    d = (rng.standard_normal((n_rows, n_cols // 256)) * 0.001).astype(np.float32)
    d[0] = np.float32(3e-7)
    d[1] = np.float32(-20.0)
    d[2] = np.float32(100.0)
    blk[:, :, 0:2] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(
        n_rows, -1, 2)
    blk[3, :, 8:] = 0x88              # codebook entry 8 (value 1) everywhere
    blk[3, :, 8 + 5] = 0x8F           # value 113 at column 5 of each block
    w = blk.reshape(-1)
    X = rng.standard_normal((T, n_cols)).astype(np.float32)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
    want = exact(oracle, t, w, X, n_rows)
    for r in range(n_rows):
        scale = np.abs(want[:, r]).max()
        assert np.abs(got[:, r] - want[:, r]).max() <= 1e-6 * scale, r


def test_split_gemm_nt4_vs_oracle(hip, oracle):
    """8192 x 4096 Q4_K with 512 tokens: 512 workgroups of 256 rows (64 rows a
    wave); tokens sampled from every 32-token tile against the oracle."""
    rng = np.random.default_rng(17)
    n_rows, n_cols, n_tok = 8192, 4096, 512
    w = W.make_table(W.Q4_K, n_rows * n_cols // 256, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    got = gpu_matmul(W.Q4_K, w, X, n_rows)
    idx = np.arange(5, n_tok, 32)
    assert rel_to_scale(got[idx], oracle.matmul(W.Q4_K, w, X[idx], n_rows)) <= RTOL


@pytest.mark.parametrize("t", [W.Q4_K, W.Q6_K])
@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (257, 4096, 100), (1000, 2048, 64), (130, 6144, 128), (64, 14336, 192)])
def test_split_gemm_64_token_tiles(hip, oracle, t, n_rows, n_cols, n_tok):
    """Workgroups of 64 tokens (AERO_HIP_TUNE gemm16_mt=4; taken by itself at
    512 tokens of gate/up or 14336-row matrices): bit-identical to the
    32-token workgroups (every accumulator sums the same products in the
    same order) and within 1e-5 of the oracle, plain and with the folded
    add + norm and the gate/up epilogue."""
    from aero_amd import device
    rng = np.random.default_rng(n_rows + n_cols + n_tok + t)
    w = table(t, n_rows, n_cols, rng)
    u = table(t, n_rows, n_cols, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    D = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (rng.standard_normal(n_cols) * 0.1 + 1).astype(np.float32)
    print(f"split gemm 64-token tiles type={t} rows={n_rows} cols={n_cols} tokens={n_tok}",
          flush=True)
    got = {}
    device.tune_set("gemm16_ksplit", 1)   # one workgroup a tile, as at the model's sizes
    try:
        for mt in (2, 4):
            device.tune_set("gemm16_mt", mt)
            plain = gpu_matmul(t, w, X, n_rows)
            out = DA.empty((n_tok, n_rows))
            xo = DA.empty((n_tok, n_cols))
            ops.norm_matmul_gate_up(t, DA.from_numpy(w), DA.from_numpy(u), DA.from_numpy(X), out,
                                    n_rows, n_cols, n_tok, act="silu", norm_w=DA.from_numpy(nw),
                                    eps=1e-5, d=DA.from_numpy(D), x_out=xo)
            got[mt] = (plain, out.numpy(), xo.numpy())
    finally:
        device.tune_set("gemm16_mt", None)
        device.tune_set("gemm16_ksplit", None)
    for a, b in zip(got[2], got[4]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert rel_to_scale(got[4][0], oracle.matmul(t, w, X, n_rows)) <= RTOL
    h = oracle.rmsnorm_rows(X + D, nw, 1e-5)
    want = oracle.act_mul(0, oracle.matmul(t, w, h, n_rows), oracle.matmul(t, u, h, n_rows))
    assert rel_to_scale(got[4][1], want) <= RTOL


@pytest.mark.parametrize("t", [W.Q6_K, W.Q8_0])
def test_split_gemm_16_row_waves(hip, oracle, t):
    """Q6_K and Q8_0 4096 x 4096 at 512 tokens take waves of 16 rows with
    64-token workgroups (512 of them): bit-identical to 32-row waves of 32
    tokens (AERO_HIP_TUNE gemm16_nt1=0, gemm16_mt=2) and, on tokens from
    every 64-token tile, within 1e-5 of the oracle."""
    from aero_amd import device
    rng = np.random.default_rng(29 + t)
    n_rows, n_cols, n_tok = 4096, 4096, 512
    bv, _ = W.BLOCK[t]
    w = W.make_table(t, n_rows * n_cols // bv, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    got = gpu_matmul(t, w, X, n_rows)
    try:
        device.tune_set("gemm16_nt1", 0)
        device.tune_set("gemm16_mt", 2)
        ref = gpu_matmul(t, w, X, n_rows)
    finally:
        device.tune_set("gemm16_nt1", None)
        device.tune_set("gemm16_mt", None)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    idx = np.arange(7, n_tok, 64)
    assert rel_to_scale(got[idx], oracle.matmul(t, w, X[idx], n_rows)) <= RTOL


def test_split_gemm_small_workspace_and_host_abi(hip, oracle):
    """A workspace below aero_hip_matmul_workspace takes the fp32 GEMM (same
    results to the tolerance); the reference-compatible aero_matmul (host
    arrays) runs the split path with its own workspace."""
    rng = np.random.default_rng(23)
    n_rows, n_cols, n_tok = 200, 2048, 64
    w = W.make_table(W.Q4_K, n_rows * n_cols // 256, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    want = oracle.matmul(W.Q4_K, w, X, n_rows)
    L = _lib.lib()
    need = int(L.aero_hip_matmul_workspace(W.Q4_K, n_cols, n_tok))
    ws = DA.empty(need // 8, np.float32)                 # half the bytes needed
    dw, dx, dy = DA.from_numpy(w), DA.from_numpy(X), DA.empty((n_tok, n_rows))
    assert L.aero_hip_matmul(W.Q4_K, dw.ptr, dw.nbytes, dx.ptr, dy.ptr, n_rows, n_cols, n_tok,
                             ws.ptr, ws.nbytes, None) == 1
    assert rel_to_scale(dy.numpy(), want) <= RTOL
    Y = native.matmul(W.Q4_K, w.tobytes(), X)
    assert rel_to_scale(Y, want) <= RTOL


def _random_split_cases(n, seed):
    rng = np.random.default_rng(seed)
    unit = {W.Q4_K: 256, W.Q5_K: 256, W.Q8_0: 256, W.Q6_K: 2048, W.IQ4_XS: 512}
    types = list(unit)
    cases = []
    for i in range(n):
        t = types[i % len(types)]
        n_cols = unit[t] * int(rng.integers(1, 9 if unit[t] < 2048 else 4))
        cases.append((i, t, int(rng.integers(1, 700)), n_cols, int(rng.integers(5, 150))))
    return cases


@pytest.mark.parametrize("i,t,n_rows,n_cols,n_tok", _random_split_cases(25, 7))
def test_split_gemm_random_shapes(hip, oracle, i, t, n_rows, n_cols, n_tok):
    """Seeded random shapes of every split-path type: 1-700 rows, 5-150
    tokens (partial tiles, column splits at the low counts), the smallest
    row widths each type takes and up to 8 of them."""
    rng = np.random.default_rng(1000 + i)
    w = table(t, n_rows, n_cols, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"random split gemm {i}: type={t} rows={n_rows} cols={n_cols} tokens={n_tok}",
          flush=True)
    got = gpu_matmul(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL
