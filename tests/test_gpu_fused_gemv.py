"""GPU parity: the fused decode GEMVs (aero_hip_norm_matvec: RMSNorm + up to
four projections sharing x; aero_hip_norm_gate_up: RMSNorm + gate/up
projections + act·mul) against the oracle's composition of the reference's
separate passes: rmsnorm_rows (src/transformer.cpp:98-104), matvec / matmul
(src/kernels.cpp:497-538) and act_mul (src/tensor.cpp:104-125).

Tolerance: 1e-5 relative to the output's scale (the reference's RTOL for fp32
ops, tests/test_transformer_native.py:34-37); the fused path sums x^2 and the
dots in other orders than the reference's serial loops.
"""
import ctypes

import numpy as np
import pytest

from conftest import RTOL, rel_to_scale
from aero_amd import _lib, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

TYPES = [W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS]
SILU, GELU, GELU_TANH, IDENT = 0, 1, 2, 3


def table(t, n_rows, n_cols, rng):
    return W.make_table(t, n_rows * n_cols // W.BLOCK[t][0], rng)


def want_proj(oracle, t, w, xn, n_rows):
    return oracle.matmul(t, w, xn, n_rows)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_tok", [1, 3])
def test_norm_matvec_qkv_vs_oracle(hip, oracle, t, n_tok):
    """Three matrices (q 512 rows, k and v 128) of 2048 columns (rows of a
    multiple of 16 bytes for every type) sharing one normalised x; 3 tokens
    run the 4-token kernel with one token idle."""
    rng = np.random.default_rng(3 * t + n_tok)
    n_cols, rows = 2048, [512, 128, 128]
    ws = [table(t, nr, n_cols, rng) for nr in rows]
    x = (rng.standard_normal((n_tok, n_cols)) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    ys = [DA.empty((n_tok, nr)) for nr in rows]
    print(f"norm_matvec type={t} tokens={n_tok}", flush=True)
    ops.norm_matvec(t, [DA.from_numpy(w) for w in ws], DA.from_numpy(x), ys, rows, n_cols,
                    n_tok, norm_w=DA.from_numpy(nw), eps=1e-5)
    xn = oracle.rmsnorm_rows(x, nw, 1e-5)
    for w, nr, y in zip(ws, rows, ys):
        assert rel_to_scale(y.numpy(), want_proj(oracle, t, w, xn, nr)) <= RTOL


@pytest.mark.parametrize("t", [W.Q4_K, W.Q8_0, W.Q6_K])
@pytest.mark.parametrize("n_tok,norm", [(1, False), (2, True), (4, False)])
def test_norm_matvec_four_matrices(hip, oracle, t, n_tok, norm):
    """Four matrices in one launch, as a DeltaNet layer's projections of x
    (qkv 1536, gate 512, alpha and beta 8 rows: the small ones one workgroup
    each) of 2048 columns; without the norm (the layer's x is already
    normed) and with it."""
    rng = np.random.default_rng(7 * t + n_tok)
    n_cols, rows = 2048, [1536, 512, 8, 8]
    ws = [table(t, nr, n_cols, rng) for nr in rows]
    x = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    ys = [DA.empty((n_tok, nr)) for nr in rows]
    print(f"norm_matvec 4 matrices type={t} tokens={n_tok} norm={norm}", flush=True)
    ops.norm_matvec(t, [DA.from_numpy(w) for w in ws], DA.from_numpy(x), ys, rows, n_cols,
                    n_tok, norm_w=DA.from_numpy(nw) if norm else None, eps=1e-5, norm=norm)
    xn = oracle.rmsnorm_rows(x, nw, 1e-5) if norm else x
    for w, nr, y in zip(ws, rows, ys):
        assert rel_to_scale(y.numpy(), want_proj(oracle, t, w, xn, nr)) <= RTOL


@pytest.mark.parametrize("t,n_cols,w_len", [(W.Q4_K, 4096, 128), (W.Q8_0, 1024, 64),
                                             (W.Q6_K, 2048, 256), (W.IQ4_XS, 512, 128)])
@pytest.mark.parametrize("n_tok", [1, 2])
def test_gated_norm_matvec_vs_oracle(hip, oracle, t, n_cols, w_len, n_tok):
    """The gated-DeltaNet norm (whole-row RMS, tiled weight, silu gate) in the
    GEMV prologue against the oracle's gated_rmsnorm_silu then matmul; one
    step of columns (512, 1024) and several (2048, 4096)."""
    rng = np.random.default_rng(n_cols + w_len + n_tok)
    n_rows = 384
    w = table(t, n_rows, n_cols, rng)
    x = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    z = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(w_len)).astype(np.float32)
    y = DA.empty((n_tok, n_rows))
    print(f"gated_norm_matvec type={t} cols={n_cols} w_len={w_len} tokens={n_tok}", flush=True)
    ops.gated_norm_matvec(t, DA.from_numpy(w), DA.from_numpy(x), DA.from_numpy(z),
                          DA.from_numpy(nw), y, n_rows, n_cols, n_tok, 1e-6)
    on = oracle.gated_rmsnorm_silu(x, z, nw, 1e-6)
    assert rel_to_scale(y.numpy(), want_proj(oracle, t, w, on, n_rows)) <= RTOL


def test_gated_norm_matvec_refusals(hip):
    rng = np.random.default_rng(5)
    w = DA.from_numpy(table(W.Q4_K, 64, 1024, rng))
    x = DA.from_numpy(rng.standard_normal((3, 1024)).astype(np.float32))
    y = DA.empty((3, 64))
    for n_tok, wl in ((3, 128), (1, 24), (1, 384)):   # 3 tokens; 24 not 16k; 384 not dividing
        nw = DA.from_numpy(np.ones(wl, np.float32))
        with pytest.raises(_lib.AeroHipError, match="gated norm"):
            ops.gated_norm_matvec(W.Q4_K, w, x, x, nw, y, 64, 1024, n_tok, 1e-6)


def test_norm_matvec_llama_decode_and_variants(hip, oracle):
    """Llama-3-8B q/k/v decode shapes (4096 -> 4096 / 1024 / 1024, Q4_K);
    without the norm the launch equals three plain GEMVs; the norm without a
    weight (ones) and with (1 + w)."""
    rng = np.random.default_rng(11)
    n_cols, rows = 4096, [4096, 1024, 1024]
    ws = [table(W.Q4_K, nr, n_cols, rng) for nr in rows]
    dws = [DA.from_numpy(w) for w in ws]
    x = rng.standard_normal((1, n_cols)).astype(np.float32)
    nw = (0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    dx, dnw = DA.from_numpy(x), DA.from_numpy(nw)
    for norm_w, unit, norm in [(dnw, False, True), (None, False, True), (dnw, True, True),
                               (None, False, False)]:
        ys = [DA.empty((1, nr)) for nr in rows]
        ops.norm_matvec(W.Q4_K, dws, dx, ys, rows, n_cols, 1, norm_w=norm_w, eps=1e-6,
                        norm=norm, unit_offset=unit)
        if norm:
            xn = oracle.rmsnorm_rows(x, None if norm_w is None else nw, 1e-6, unit_offset=unit)
        else:
            xn = x
        for w, nr, y in zip(ws, rows, ys):
            assert rel_to_scale(y.numpy(), want_proj(oracle, W.Q4_K, w, xn, nr)) <= RTOL
        if not norm:
            for w, nr, y in zip(dws, rows, ys):
                plain = DA.empty((1, nr))
                ops.matvec(W.Q4_K, w, dx, plain, nr, n_cols, 1)
                assert rel_to_scale(y.numpy(), plain.numpy()) <= RTOL


@pytest.mark.parametrize("t", [W.Q4_K, W.Q6_K])
def test_norm_matvec_two_steps(hip, oracle, t):
    """8192-column rows (two 4096-column steps, the pipelined kernel), 2 tokens."""
    rng = np.random.default_rng(21 + t)
    n_cols, rows = 8192, [300, 77]
    ws = [table(t, nr, n_cols, rng) for nr in rows]
    x = rng.standard_normal((2, n_cols)).astype(np.float32)
    nw = rng.standard_normal(n_cols).astype(np.float32)
    ys = [DA.empty((2, nr)) for nr in rows]
    ops.norm_matvec(t, [DA.from_numpy(w) for w in ws], DA.from_numpy(x), ys, rows, n_cols, 2,
                    norm_w=DA.from_numpy(nw), eps=1e-5)
    xn = oracle.rmsnorm_rows(x, nw, 1e-5)
    for w, nr, y in zip(ws, rows, ys):
        assert rel_to_scale(y.numpy(), want_proj(oracle, t, w, xn, nr)) <= RTOL


@pytest.mark.parametrize("act", [SILU, GELU, GELU_TANH, IDENT])
@pytest.mark.parametrize("t", [W.Q4_K, W.Q8_0, W.Q6_K])
def test_norm_gate_up_vs_oracle(hip, oracle, act, t):
    """act(gate . xn) * (up . xn) for 5 tokens (launches of 4 and 1), 700
    rows (partial workgroups), against the composition of the oracle's ops."""
    rng = np.random.default_rng(31 + act + 7 * t)
    n_ff, n_cols, n_tok = 700, 2048, 5
    wg, wu = table(t, n_ff, n_cols, rng), table(t, n_ff, n_cols, rng)
    x = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    out = DA.empty((n_tok, n_ff))
    ops.norm_gate_up(t, DA.from_numpy(wg), DA.from_numpy(wu), DA.from_numpy(x), out, n_ff,
                     n_cols, n_tok, act=act, norm_w=DA.from_numpy(nw), eps=1e-5)
    xn = oracle.rmsnorm_rows(x, nw, 1e-5)
    g = oracle.matmul(t, wg, xn, n_ff)
    u = oracle.matmul(t, wu, xn, n_ff)
    assert rel_to_scale(out.numpy(), oracle.act_mul(act, g, u)) <= RTOL


def test_norm_gate_up_llama_decode(hip, oracle):
    """Llama-3-8B SwiGLU decode (14336 x 4096 Q4_K gate and up, one token)
    equals rmsnorm -> two GEMVs -> act_mul on the device and the oracle."""
    rng = np.random.default_rng(41)
    n_ff, n_cols = 14336, 4096
    wg, wu = table(W.Q4_K, n_ff, n_cols, rng), table(W.Q4_K, n_ff, n_cols, rng)
    x = rng.standard_normal((1, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32)
    dwg, dwu, dx, dnw = (DA.from_numpy(a) for a in (wg, wu, x, nw))
    out = DA.empty((1, n_ff))
    ops.norm_gate_up(W.Q4_K, dwg, dwu, dx, out, n_ff, n_cols, 1, act="silu", norm_w=dnw,
                     eps=1e-5)
    xn = oracle.rmsnorm_rows(x, nw, 1e-5)
    want = oracle.act_mul(SILU, oracle.matmul(W.Q4_K, wg, xn, n_ff),
                          oracle.matmul(W.Q4_K, wu, xn, n_ff))
    assert rel_to_scale(out.numpy(), want) <= RTOL
    h, g, u, o = DA.empty((1, n_cols)), DA.empty((1, n_ff)), DA.empty((1, n_ff)), DA.empty((1, n_ff))
    ops.rmsnorm(dx, dnw, h, 1, n_cols, 1e-5)
    ops.matvec(W.Q4_K, dwg, h, g, n_ff, n_cols, 1)
    ops.matvec(W.Q4_K, dwu, h, u, n_ff, n_cols, 1)
    ops.act_mul("silu", g, u, o)
    assert rel_to_scale(out.numpy(), o.numpy()) <= RTOL


def test_fused_refusals(hip):
    """Five matrices, a type without a GEMV, misaligned weights, rows not a
    multiple of 16 bytes (Q6_K at 1024 columns: 840 bytes; Q8_0 rows of 952
    bytes in an odd number) and gate/up of different sizes are refused with
    an error, nothing launched."""
    rng = np.random.default_rng(51)
    w = DA.from_numpy(table(W.Q4_K, 64, 1024, rng))
    x = DA.from_numpy(rng.standard_normal((1, 1024)).astype(np.float32))
    ys = [DA.empty((1, 64)) for _ in range(5)]
    with pytest.raises(ValueError):
        ops.norm_matvec(W.Q4_K, [w] * 5, x, ys, [64] * 5, 1024)
    L = _lib.lib()
    p5 = (ctypes.c_void_p * 5)(*[w.ptr] * 5)
    b5 = (ctypes.c_int64 * 5)(*[w.nbytes] * 5)
    r5 = (ctypes.c_int64 * 5)(*[64] * 5)
    y5 = (ctypes.c_void_p * 5)(*[y.ptr for y in ys])
    assert L.aero_hip_norm_matvec(W.Q4_K, 5, p5, b5, r5, y5, x.ptr, None, 1e-5, 0, 1024, 1,
                                  None) == 0
    assert "n_mat=5" in _lib.last_error()
    with pytest.raises(_lib.AeroHipError):
        ops.norm_matvec(W.F32, [w], x, ys[:1], [64], 1024)
    w6 = DA.from_numpy(table(W.Q6_K, 64, 1024, rng))
    with pytest.raises(_lib.AeroHipError, match="whole 16 bytes"):
        ops.norm_matvec(W.Q6_K, [w6], x, ys[:1], [64], 1024)
    # Q8_0 rows of 952 bytes: an odd row count ends 8 bytes short of a
    # 16-byte boundary, which the last lane window would read past the weights
    w8 = DA.from_numpy(table(W.Q8_0, 127, 896, rng))
    x8 = DA.from_numpy(rng.standard_normal((1, 896)).astype(np.float32))
    with pytest.raises(_lib.AeroHipError, match="window"):
        ops.norm_matvec(W.Q8_0, [w8], x8, [DA.empty((1, 127))], [127], 896)
    L = _lib.lib()
    wp = (ctypes.c_void_p * 1)(w.ptr + 4)                    # 4-byte aligned only
    wb = (ctypes.c_int64 * 1)(w.nbytes - 4)
    nr = (ctypes.c_int64 * 1)(32)
    yp = (ctypes.c_void_p * 1)(ys[0].ptr)
    assert L.aero_hip_norm_matvec(W.Q4_K, 1, wp, wb, nr, yp, x.ptr, None, 1e-5, 0, 1024, 1,
                                  None) == 0
    assert "aligned" in _lib.last_error()
    w2 = DA.from_numpy(table(W.Q4_K, 32, 1024, rng))
    with pytest.raises(ValueError):
        ops.norm_gate_up(W.Q4_K, w, w2, x, DA.empty((1, 64)), 64, 1024)
    with pytest.raises(_lib.AeroHipError):                    # 64 rows need 64 * 576 bytes
        ops.norm_gate_up(W.Q4_K, w2, w2, x, DA.empty((1, 64)), 64, 1024)


@pytest.mark.parametrize("n_tok", [1, 3])
def test_fused_q8_0_qwen2_0p5b_rows(hip, oracle, n_tok):
    """Qwen2-0.5B's decode projections in Q8_0 (896 columns: 952-byte rows,
    every other one 8 bytes off a 16-byte boundary): RMSNorm + q/k/v (896,
    128, 128 rows) and RMSNorm + gate/up (4864) + SiLU·mul in one launch
    each, against the oracle's rmsnorm -> matmul (-> act_mul)."""
    rng = np.random.default_rng(91 + n_tok)
    N, F = 896, 4864
    x = rng.standard_normal((n_tok, N)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    rows = (896, 128, 128)
    mats = [table(W.Q8_0, r, N, rng) for r in rows]
    dx, dw = DA.from_numpy(x), DA.from_numpy(nw)
    ys = [DA.empty((n_tok, r)) for r in rows]
    print(f"fused Q8_0 896 tokens={n_tok}", flush=True)
    ops.norm_matvec(W.Q8_0, [DA.from_numpy(m) for m in mats], dx, ys, list(rows), N, n_tok,
                    norm_w=dw, eps=1e-6)
    xn = oracle.rmsnorm_rows(x, nw, 1e-6)
    for y, m, r in zip(ys, mats, rows):
        assert rel_to_scale(y.numpy(), want_proj(oracle, W.Q8_0, m, xn, r)) <= RTOL
    wg, wu = table(W.Q8_0, F, N, rng), table(W.Q8_0, F, N, rng)
    out = DA.empty((n_tok, F))
    ops.norm_gate_up(W.Q8_0, DA.from_numpy(wg), DA.from_numpy(wu), dx, out, F, N, n_tok,
                     act="silu", norm_w=dw, eps=1e-6)
    want = oracle.act_mul(SILU, oracle.matmul(W.Q8_0, wg, xn, F),
                          oracle.matmul(W.Q8_0, wu, xn, F))
    assert rel_to_scale(out.numpy(), want) <= RTOL
