"""GPU parity: the quantised GEMV / small-batch GEMM (aero_hip_matvec) and the
reference-compatible aero_matvec / aero_matmul, against the oracle's
restatement of src/kernels.cpp:78-250,497-538 and the reference's own outputs
(tests/golden/ref_vectors.npz). The GPU sums in a different order from the
reference's serial loops, so results agree to a tolerance relative to the
output's scale: 1e-5 (observed ~1e-7), the reference's own RTOL for fp32 ops
(tests/test_transformer_native.py:34-37).
"""
import numpy as np
import pytest

from conftest import RTOL, golden, rel_to_scale
from aero_amd import native, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

TYPES = [W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS]


def gpu_matvec(t, w, X, n_rows):
    X = np.atleast_2d(np.ascontiguousarray(X, np.float32))
    T, n_cols = X.shape
    y = DA.empty((T, n_rows))
    ops.matvec(t, DA.from_numpy(w), DA.from_numpy(X), y, n_rows, n_cols, T)
    return y.numpy()


@pytest.mark.parametrize("t", TYPES)
def test_matvec_golden(hip, t):
    """The reference's own matvec / matmul outputs (24 x 512, 3 tokens)."""
    g = golden("ref_vectors.npz")
    w, X = g[f"mv{t}_w"], g[f"mv{t}_x"]
    n_rows = g[f"mv{t}_y"].size
    assert rel_to_scale(gpu_matvec(t, w, X[:1], n_rows)[0], g[f"mv{t}_y"]) <= RTOL
    assert rel_to_scale(gpu_matvec(t, w, X, n_rows), g[f"mm{t}_y"]) <= RTOL


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (1, 256, 1), (37, 1024, 1), (4096, 4096, 1), (1000, 14336, 1),   # decode shapes
    (4103, 4096, 2), (513, 2048, 3), (130, 4096, 8), (67, 1024, 13),  # token groups
    (300, 14336, 5), (64, 8192, 4),  # rows of several 4096-column steps, token groups
    # 5-24 tokens: Q4_K / Q5_K take the split GEMM (5+ tokens from 32M
    # weights, 12+ from 8M, else 16+), the other types the GEMV
    (8200, 1024, 8), (100, 2048, 16), (33, 512, 24), (8192, 4096, 5),
])
def test_matvec_vs_oracle(hip, oracle, t, n_rows, n_cols, n_tok):
    rng = np.random.default_rng(n_rows * 31 + n_cols + n_tok + t)
    bv, bb = W.BLOCK[t]
    w = W.make_table(t, n_rows * n_cols // bv, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"matvec type={t} rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    got = gpu_matvec(t, w, X, n_rows)
    want = oracle.matmul(t, w, X, n_rows)
    assert rel_to_scale(got, want) <= RTOL


@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (896, 896, 1), (128, 896, 3), (4864, 896, 1), (127, 896, 2), (64, 640, 5),
])
def test_matvec_q8_0_rows_of_8_bytes(hip, oracle, n_rows, n_cols, n_tok):
    """Q8_0 rows of a multiple of 8 bytes but not of 16 (896 columns: 952
    bytes, Qwen2-0.5B; 640: 680) alternate between 16- and 8-byte aligned
    starts: the 64-column lane kernel places each lane's 16-byte window from
    the absolute address. With an odd row count the last row ends 8 bytes
    short of a 16-byte boundary, past the weights: that matrix takes the
    word kernel. Both match the oracle."""
    t = W.Q8_0
    rng = np.random.default_rng(n_rows + n_cols + n_tok)
    w = W.make_table(t, n_rows * n_cols // 32, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"matvec Q8_0 rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    assert rel_to_scale(gpu_matvec(t, w, X, n_rows), oracle.matmul(t, w, X, n_rows)) <= RTOL


@pytest.mark.parametrize("t", [W.Q8_0, W.Q6_K])
def test_matvec_rows_off_word_boundary(hip, oracle, t):
    """Row sizes that are not a multiple of 4 bytes (Q8_0 with 45 blocks per row,
    Q6_K with 5): every other row starts 2 bytes past a 4-byte word."""
    rng = np.random.default_rng(61 + t)
    bv, bb = W.BLOCK[t]
    nb = 45 if t == W.Q8_0 else 5
    n_rows, n_cols = 301, nb * bv
    assert (nb * bb) % 4 == 2
    w = W.make_table(t, n_rows * nb, rng)
    X = rng.standard_normal((3, n_cols)).astype(np.float32)
    assert rel_to_scale(gpu_matvec(t, w, X, n_rows), oracle.matmul(t, w, X, n_rows)) <= RTOL


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_rows,n_cols,n_tok", [
    (100, 1024, 40), (130, 2048, 33), (257, 4096, 100), (64, 14336, 64),
])
def test_matmul_many_tokens_vs_oracle(hip, oracle, t, n_rows, n_cols, n_tok):
    """32 or more tokens take the matrix-core GEMM (64 x 64 tiles, partial
    row and token tiles, rows of 1 to 56 blocks)."""
    rng = np.random.default_rng(n_rows * 17 + n_cols + n_tok + t)
    bv, bb = W.BLOCK[t]
    w = W.make_table(t, n_rows * n_cols // bv, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    print(f"matmul type={t} rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    got = gpu_matvec(t, w, X, n_rows)
    want = oracle.matmul(t, w, X, n_rows)
    assert rel_to_scale(got, want) <= RTOL


def test_matmul_prefill_size_matches_gemv(hip):
    """At Llama-3-8B FFN size with 512 tokens (14336 x 4096 Q4_K, the prefill
    shape), every token's GEMM row equals that token's GEMV (one-token launch)
    to the tolerance; sampled tokens cover every 64-token tile."""
    rng = np.random.default_rng(91)
    n_rows, n_cols, n_tok = 14336, 4096, 512
    w = W.make_table(W.Q4_K, n_rows * n_cols // 256, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    Y = gpu_matvec(W.Q4_K, w, X, n_rows)
    for i in (0, 63, 64, 200, 383, 511):
        assert rel_to_scale(Y[i], gpu_matvec(W.Q4_K, w, X[i], n_rows)[0]) <= RTOL


def test_matvec_linearity_at_full_size(hip):
    """At Llama-3-8B FFN-down size (4096 x 14336 Q4_K): W(a*x1 + x2) equals
    a*W(x1) + W(x2) to the tolerance, and a zero x gives exactly zero."""
    rng = np.random.default_rng(71)
    n_rows, n_cols = 4096, 14336
    w = W.make_table(W.Q4_K, n_rows * n_cols // 256, rng)
    x1, x2 = rng.standard_normal((2, n_cols)).astype(np.float32)
    a = np.float32(0.75)
    X = np.stack([x1, x2, a * x1 + x2, np.zeros(n_cols, np.float32)])
    Y = gpu_matvec(W.Q4_K, w, X, n_rows).astype(np.float64)
    assert rel_to_scale(Y[2], a * Y[0] + Y[1]) <= RTOL
    assert not Y[3].any()


def test_host_abi_matvec_matmul(hip, oracle):
    """engine/native.py-shaped calls (host arrays, bytes) and the reference's
    refusals (tests/test_kernels.cpp:242-250)."""
    rng = np.random.default_rng(81)
    for t in TYPES:
        bv, bb = W.BLOCK[t]
        n_rows, n_cols = 29, 4 * 256
        w = W.make_table(t, n_rows * n_cols // bv, rng)
        x = rng.standard_normal(n_cols).astype(np.float32)
        X = rng.standard_normal((5, n_cols)).astype(np.float32)
        y = native.matvec(t, w.tobytes(), x)
        assert y.shape == (n_rows,)
        assert rel_to_scale(y, oracle.matvec(t, w, x, n_rows)) <= RTOL
        Y = native.matmul(t, bytearray(w.tobytes()), X)
        assert Y.shape == (5, n_rows)
        assert rel_to_scale(Y, oracle.matmul(t, w, X, n_rows)) <= RTOL
    with pytest.raises(ValueError):
        native.matvec(W.F32, bytes(64), np.zeros(16, np.float32))
    with pytest.raises(ValueError):
        native.matvec(W.Q4_K, bytes(144 * 4), np.zeros(255, np.float32))


@pytest.mark.parametrize("t", [W.Q4_K, W.Q8_0, W.Q6_K, W.IQ4_XS, W.Q5_K])
@pytest.mark.parametrize("n_rows,n_cols", [(1, 2048), (3, 1024), (37, 2048), (129, 512)])
@pytest.mark.parametrize("n_tok", [1, 2, 4])
def test_matvec_half_wave_rows(hip, oracle, t, n_rows, n_cols, n_tok):
    """Rows of at most 2048 columns, one a half-wave: odd row counts leave the
    last wave's upper half on a clamped row whose sum is not stored, and rows
    of 512 columns use 8 of a half-wave's 32 column slots."""
    rng = np.random.default_rng(n_rows * 7 + n_cols + n_tok + t)
    w = W.make_table(t, n_rows * n_cols // W.BLOCK[t][0], rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    got = gpu_matvec(t, w, X, n_rows)
    assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL


@pytest.mark.parametrize("n_tok", [1, 3])
def test_norm_matvec_half_wave_odd_rows(hip, oracle, n_tok):
    """The fused decode GEMV over three matrices of odd row counts and 2048
    columns (a row a half-wave), with the RMSNorm in its prologue."""
    t, n_cols, rows = W.Q4_K, 2048, [37, 5, 1]
    rng = np.random.default_rng(61 + n_tok)
    ws = [W.make_table(t, r * n_cols // 256, rng) for r in rows]
    x = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    ys = [DA.empty((n_tok, r)) for r in rows]
    ops.norm_matvec(t, [DA.from_numpy(w) for w in ws], DA.from_numpy(x), ys, rows, n_cols,
                    n_tok, norm_w=DA.from_numpy(nw), eps=1e-5)
    h = oracle.rmsnorm_rows(x, nw, 1e-5)
    for w, r, y in zip(ws, rows, ys):
        assert rel_to_scale(y.numpy(), oracle.matmul(t, w, h, r)) <= RTOL
