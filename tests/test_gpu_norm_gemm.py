"""GPU parity: the prefill norm -> projection forms (aero_hip_norm_matmul,
aero_hip_norm_matmul_gate_up) against the oracle's composition of the passes
they replace: the residual add `x_ += o_` and norm_row (src/model.cpp:244-245,
279-282), matmul (src/kernels.cpp:520-538) and act_mul (src/model.cpp:172-175).

Q4_K / Q5_K with 32+ tokens take the split-x GEMM with the add and the norm
folded into its pre-pass and act(gate)*up in its epilogue; below 32 tokens
rows of whole 16 bytes take the fused decode GEMV (the add and the norm in its
prologue, act(gate)*up in its epilogue); other types and token counts take
separate launches. Tolerance: 1e-5 of the output's scale
(the reference's RTOL, tests/test_transformer_native.py:34-37); the residual
stream x + d is bit-exact (one IEEE add).
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import _lib, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

ACT = {"silu": 0, "gelu": 1, "gelu_tanh": 2}


def weights(t, n_rows, n_cols, rng):
    return W.make_table(t, n_rows * n_cols // W.BLOCK[t][0], rng)


def oracle_h(oracle, x, d, w, eps, unit_offset, norm=True):
    xs = x + d if d is not None else x
    return xs, (oracle.rmsnorm_rows(xs, w, eps, unit_offset) if norm else xs)


@pytest.mark.parametrize("t", [W.Q4_K, W.Q5_K, W.Q6_K, W.Q8_0])
@pytest.mark.parametrize("n_tok,n_cols,rows", [
    (64, 1024, (256, 64, 64)), (33, 2048, (130,)), (100, 512, (96, 40)), (7, 1024, (64, 64, 64)),
    (2, 1024, (64, 64, 64)), (1, 5120, (96, 32)),
])
@pytest.mark.parametrize("form", ["norm", "resid_norm", "unit_offset", "no_norm",
                                  "resid_no_norm"])
def test_norm_matmul_vs_oracle(hip, oracle, t, n_tok, n_cols, rows, form):
    rng = np.random.default_rng(n_tok * 7 + n_cols + len(rows) + t)
    x = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    d = (rng.standard_normal((n_tok, n_cols), dtype=np.float32)
         if form.startswith("resid") else None)
    uo = form == "unit_offset"
    w = (rng.standard_normal(n_cols, dtype=np.float32) * np.float32(0.1) + (0 if uo else 1)
         ).astype(np.float32)
    mats = [weights(t, r, n_cols, rng) for r in rows]
    print(f"norm_matmul type={t} tok={n_tok} cols={n_cols} rows={rows} form={form}", flush=True)
    dx, dw = DA.from_numpy(x), DA.from_numpy(w)
    dd = None if d is None else DA.from_numpy(d)
    ys = [DA.empty((n_tok, r)) for r in rows]
    norm = not form.endswith("no_norm")
    ops.norm_matmul(t, [DA.from_numpy(m) for m in mats], dx, ys, list(rows), n_cols, n_tok,
                    norm_w=dw, eps=1e-5, norm=norm, unit_offset=uo, d=dd)
    xs, h = oracle_h(oracle, x, d, w, 1e-5, uo, norm=norm)
    if d is not None:
        assert bits_equal(dx.numpy(), xs)          # the residual stream, in place
    for y, m, r in zip(ys, mats, rows):
        assert rel_to_scale(y.numpy(), oracle.matmul(t, m, h, r)) <= RTOL


@pytest.mark.parametrize("t", [W.Q4_K, W.Q8_0, W.Q5_K, W.Q6_K, W.IQ4_XS])
@pytest.mark.parametrize("n_tok,n_cols,rows", [
    (1, 4096, (512, 128, 128)), (3, 1024, (64, 96)), (5, 8192, (96,)), (2, 5120, (64, 32, 64)),
    (31, 512, (64,)), (1, 5120, (64, 32, 64)), (1, 8192, (96,)),
])
@pytest.mark.parametrize("apart", [True, False])
def test_norm_matmul_resid_few_tokens(hip, oracle, t, n_tok, n_cols, rows, apart):
    """Below 32 tokens, rows of whole 16 bytes take the fused decode GEMV: at
    one token with x_out apart from x and d, with the add and the norm in its
    prologue (one workgroup stores x + d); else after an add + norm pass.
    Rows of other sizes (Q6_K here at 1024 and 5120 columns) take add + norm
    then the GEMVs. All match the oracle, and x_out is x + d bit for bit."""
    rng = np.random.default_rng(n_tok * 13 + n_cols + len(rows) + t)
    x = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    d = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    w = (rng.standard_normal(n_cols, dtype=np.float32) * np.float32(0.1) + 1).astype(np.float32)
    mats = [weights(t, r, n_cols, rng) for r in rows]
    print(f"norm_matmul few tokens type={t} tok={n_tok} cols={n_cols} rows={rows} "
          f"apart={apart}", flush=True)
    dx, dd, dw = DA.from_numpy(x), DA.from_numpy(d), DA.from_numpy(w)
    xo = DA.empty(x.shape) if apart else dx
    ys = [DA.empty((n_tok, r)) for r in rows]
    ops.norm_matmul(t, [DA.from_numpy(m) for m in mats], dx, ys, list(rows), n_cols, n_tok,
                    norm_w=dw, eps=1e-5, d=dd, x_out=xo)
    xs, h = oracle_h(oracle, x, d, w, 1e-5, False)
    assert bits_equal(xo.numpy(), xs)
    if apart:
        assert bits_equal(dx.numpy(), x)
    for y, m, r in zip(ys, mats, rows):
        assert rel_to_scale(y.numpy(), oracle.matmul(t, m, h, r)) <= RTOL


@pytest.mark.parametrize("t", [W.Q4_K, W.Q5_K, W.Q6_K, W.Q8_0, W.IQ4_XS])
@pytest.mark.parametrize("act", list(ACT))
@pytest.mark.parametrize("n_tok,n_cols,n_ff", [(64, 1024, 320), (45, 512, 100), (5, 512, 64),
                                              (1, 5120, 96), (3, 8192, 64), (40, 2048, 96)])
def test_gate_up_vs_oracle(hip, oracle, t, act, n_tok, n_cols, n_ff):
    rng = np.random.default_rng(n_tok + n_cols + n_ff + t + ACT[act])
    x = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    d = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    w = (np.float32(1) + rng.standard_normal(n_cols, dtype=np.float32) * np.float32(0.1))
    wg, wu = weights(t, n_ff, n_cols, rng), weights(t, n_ff, n_cols, rng)
    print(f"gate_up type={t} act={act} tok={n_tok} cols={n_cols} ff={n_ff}", flush=True)
    dx, dd = DA.from_numpy(x), DA.from_numpy(d)
    xo = DA.empty(x.shape)
    out = DA.empty((n_tok, n_ff))
    ops.norm_matmul_gate_up(t, DA.from_numpy(wg), DA.from_numpy(wu), dx, out, n_ff, n_cols,
                            n_tok, act=act, norm_w=DA.from_numpy(w), eps=1e-6, d=dd, x_out=xo)
    xs, h = oracle_h(oracle, x, d, w, 1e-6, False)
    assert bits_equal(xo.numpy(), xs)
    assert bits_equal(dx.numpy(), x)                # x untouched when x_out is separate
    g = oracle.matmul(t, wg, h, n_ff)
    u = oracle.matmul(t, wu, h, n_ff)
    assert rel_to_scale(out.numpy(), oracle.act_mul(ACT[act], g, u)) <= RTOL


def exact_rows(oracle, t, mat, n_cols, rows, h):
    """float64 h @ W[rows]^T over the oracle's dequantised rows."""
    bv, bb = W.BLOCK[t]
    rb = n_cols // bv * bb
    Wd = np.stack([oracle.dequant(t, mat[r * rb:(r + 1) * rb], n_cols) for r in rows])
    return h.astype(np.float64) @ Wd.astype(np.float64).T


def test_llama3_8b_prefill_layer_shapes(hip, oracle):
    """512 tokens of 4096: q/k/v (4096, 1024, 1024 rows) after add+norm, and
    gate/up (14336) + SwiGLU. Every output against the unfused GPU passes
    (add_rmsnorm, the split GEMM, act_mul), and 256 sampled rows of each
    against the float64 product of the oracle's dequantised weights."""
    s = W.SHAPES["llama3_8b_prefill"]
    T, N, F = s.n_tok, s.hidden, s.ffn
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, N), dtype=np.float32)
    d = rng.standard_normal((T, N), dtype=np.float32)
    w = np.float32(1) + rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)
    dw = DA.from_numpy(w)
    xs, h = oracle_h(oracle, x, d, w, s.eps, False)
    # q/k/v
    rows = (s.hq * s.head_dim, s.hk * s.head_dim, s.hk * s.head_dim)
    mats = [weights(W.Q4_K, r, N, rng) for r in rows]
    dmats = [DA.from_numpy(m) for m in mats]
    dx, dd = DA.from_numpy(x), DA.from_numpy(d)
    ys = [DA.empty((T, r)) for r in rows]
    print("llama3 qkv", flush=True)
    ops.norm_matmul(W.Q4_K, dmats, dx, ys, list(rows), N, T, norm_w=dw, eps=s.eps, d=dd)
    assert bits_equal(dx.numpy(), xs)
    hb = DA.empty((T, N))
    ops.rmsnorm(DA.from_numpy(xs), dw, hb, T, N, s.eps)
    for y, dm, m, r in zip(ys, dmats, mats, rows):
        ref = DA.empty((T, r))
        ops.matvec(W.Q4_K, dm, hb, ref, r, N, T)
        got = y.numpy()
        assert rel_to_scale(got, ref.numpy()) <= RTOL
        pick = np.sort(rng.choice(r, 256, replace=False))
        assert rel_to_scale(got[:, pick], exact_rows(oracle, W.Q4_K, m, N, pick, h)) <= RTOL
    # gate/up + SwiGLU
    print("llama3 gate/up", flush=True)
    wg, wu = weights(W.Q4_K, F, N, rng), weights(W.Q4_K, F, N, rng)
    dg, du = DA.from_numpy(wg), DA.from_numpy(wu)
    out = DA.empty((T, F))
    dx2 = DA.from_numpy(x)
    ops.norm_matmul_gate_up(W.Q4_K, dg, du, dx2, out, F, N, T, act="silu", norm_w=dw,
                            eps=s.eps, d=dd)
    assert bits_equal(dx2.numpy(), xs)
    g, u = DA.empty((T, F)), DA.empty((T, F))
    ops.matvec(W.Q4_K, dg, hb, g, F, N, T)
    ops.matvec(W.Q4_K, du, hb, u, F, N, T)
    ops.act_mul("silu", g, u, g)
    got = out.numpy()
    assert rel_to_scale(got, g.numpy()) <= RTOL
    pick = np.sort(rng.choice(F, 256, replace=False))
    gx = exact_rows(oracle, W.Q4_K, wg, N, pick, h)
    ux = exact_rows(oracle, W.Q4_K, wu, N, pick, h)
    with np.errstate(over="ignore"):          # exp(-g) -> inf: silu(g) -> 0
        want = (gx / (1.0 + np.exp(-gx))) * ux
    assert rel_to_scale(got[:, pick], want) <= RTOL


def test_norm_matmul_refusals(hip):
    """Refused on the host before any launch: no or too small a workspace,
    d without x_out, a misaligned x."""
    L = _lib.lib()
    n_tok, n_cols, n_rows = 64, 512, 64
    need = L.aero_hip_norm_matmul_workspace(W.Q4_K, n_cols, 0, n_tok)
    assert need > 0
    x = DA.empty((n_tok, n_cols))
    y = DA.empty((n_tok, n_rows))
    m = DA.empty((n_rows * n_cols // 256 * 144,), np.uint8)
    import ctypes
    wp = (ctypes.c_void_p * 1)(m.ptr)
    wb = (ctypes.c_int64 * 1)(m.nbytes)
    nr = (ctypes.c_int64 * 1)(n_rows)
    yp = (ctypes.c_void_p * 1)(y.ptr)
    ws = DA.empty((need,), np.uint8)
    args = lambda xp, d, xo, wsp, wsb: (W.Q4_K, 1, wp, wb, nr, yp, xp, d, xo, None, 1e-5, 0,  # noqa: E731
                                        n_cols, n_tok, wsp, wsb, None)
    assert L.aero_hip_norm_matmul(*args(x.ptr, None, None, None, 0)) == 0
    assert "workspace" in _lib.last_error()
    assert L.aero_hip_norm_matmul(*args(x.ptr, None, None, ws.ptr, need - 256)) == 0
    assert L.aero_hip_norm_matmul(*args(x.ptr, x.ptr, None, ws.ptr, need)) == 0
    assert L.aero_hip_norm_matmul(*args(x.ptr + 4, None, None, ws.ptr, need)) == 0
    assert L.aero_hip_norm_matmul(*args(x.ptr, None, None, ws.ptr, need)) == 1
    # gate/up weights off a 16-byte boundary take the separate launches,
    # whose h and up buffers this split-sized workspace cannot hold
    n_ff = 64
    need_gu = L.aero_hip_norm_matmul_workspace(W.Q4_K, n_cols, n_ff, n_tok)
    assert need_gu < n_tok * (n_cols + n_ff) * 4
    ws_gu = DA.empty((need_gu,), np.uint8)
    m2 = DA.empty((2 * m.nbytes + 16,), np.uint8)
    out = DA.empty((n_tok, n_ff))
    assert L.aero_hip_norm_matmul_gate_up(W.Q4_K, m2.ptr + 4, m2.ptr + 4 + m.nbytes, m.nbytes,
                                          x.ptr, None, None, None, 1e-5, 0, 0, out.ptr, n_ff,
                                          n_cols, n_tok, ws_gu.ptr, need_gu, None) == 0
    assert "workspace" in _lib.last_error()


@pytest.mark.parametrize("t,n_tok,n_cols,head_dim,n_heads,mode,resid,n_rope", [
    # one token: the fused GEMV's prologue (add + norm) and RoPE epilogue
    (W.Q4_K, 1, 4096, 128, (4, 2, 2), 0, True, 2),
    (W.Q4_K, 1, 4096, 128, (4, 2, 2), 1, False, 2),
    (W.Q8_0, 1, 1024, 64, (4, 2, 2), 0, True, 1),
    (W.Q4_K, 1, 5120, 128, (2, 1), 0, True, 2),          # two-step rows
    (W.IQ4_XS, 2, 1024, 64, (3, 1, 1), 0, False, 2),     # two tokens, norm in the prologue
    (W.Q5_K, 3, 2048, 128, (2, 1, 1), 0, True, 2),       # add + norm pass, RoPE epilogue
    (W.Q4_K, 4, 1024, 64, (4, 2, 2), 1, True, 2),        # four tokens: 4 rows a wave
    (W.Q4_K, 5, 8192, 128, (2, 1, 1), 0, False, 2),
    (W.Q4_K, 1, 1024, 48, (4, 2, 2), 0, True, 2),        # heads of 48 rows, 6 workgroups a head
    (W.Q4_K, 1, 1024, 40, (4, 2, 2), 0, True, 2),        # NeoX heads of 40 rows: RoPE pass
    (W.Q6_K, 2, 1024, 64, (2, 1, 1), 0, True, 2),        # 840-byte rows: separate launches
    (W.Q4_K, 40, 1024, 128, (2, 1, 1), 0, True, 2),      # split GEMM, then the RoPE pass
    (W.Q8_0, 1, 896, 64, (14, 2, 2), 0, True, 2),        # Qwen2-0.5B: 952-byte rows
])
def test_norm_matmul_rope_vs_oracle(hip, oracle, t, n_tok, n_cols, head_dim, n_heads, mode,
                                    resid, n_rope):
    """aero_hip_norm_matmul_rope: the projections of the norm (and residual
    add), then RoPE over every channel of the first n_rope outputs (q, k)
    at the tokens' positions, against the oracle's rmsnorm -> matmul ->
    qk_norm_rope (src/attention_layer.cpp:60-156 without the head norms).
    The fused decode GEMV rotates in its epilogue (NeoX partners 64 rows
    apart meet in LDS); other paths run the RoPE pass; both to 1e-5."""
    rng = np.random.default_rng(n_tok * 31 + n_cols + head_dim + mode + t)
    rows = tuple(h * head_dim for h in n_heads)
    x = rng.standard_normal((n_tok, n_cols), dtype=np.float32)
    d = rng.standard_normal((n_tok, n_cols), dtype=np.float32) if resid else None
    w = (rng.standard_normal(n_cols, dtype=np.float32) * np.float32(0.1) + 1).astype(np.float32)
    mats = [weights(t, r, n_cols, rng) for r in rows]
    pos = rng.integers(0, 16384, n_tok).astype(np.int32)
    theta = 500000.0
    n_rot, inv = ops.rope_inv_freq(head_dim, None, theta)
    assert n_rot == head_dim
    print(f"norm_matmul_rope type={t} tok={n_tok} cols={n_cols} D={head_dim} heads={n_heads} "
          f"mode={mode} resid={resid} n_rope={n_rope}", flush=True)
    dx, dw = DA.from_numpy(x), DA.from_numpy(w)
    dd = None if d is None else DA.from_numpy(d)
    xo = DA.empty(x.shape) if resid else None
    ys = [DA.empty((n_tok, r)) for r in rows]
    rope = {"n": n_rope, "head_dim": head_dim, "mode": mode, "pos": DA.from_numpy(pos),
            "inv_freq": DA.from_numpy(inv)}
    ops.norm_matmul(t, [DA.from_numpy(m) for m in mats], dx, ys, list(rows), n_cols, n_tok,
                    norm_w=dw, eps=1e-5, d=dd, x_out=xo, rope=rope)
    xs, h = oracle_h(oracle, x, d, w, 1e-5, False)
    if resid:
        assert bits_equal(xo.numpy(), xs)
    # the fold adds no launch; the RoPE pass adds one
    from aero_amd.device import Plan
    rb = n_cols // W.BLOCK[t][0] * W.BLOCK[t][1]
    lanes = rb % 16 == 0 or (t == W.Q8_0 and rb % 8 == 0 and
                             all(r * rb % 16 == 0 for r in rows))
    folds = n_tok < 32 and lanes and (mode == 1 or head_dim % 16 == 0)
    dmats = [DA.from_numpy(mm) for mm in mats]
    counts = []
    for rp in (None, rope):
        plan = Plan()
        with plan:
            ops.norm_matmul(t, dmats, dx, [DA.empty((n_tok, r)) for r in rows], list(rows),
                            n_cols, n_tok, norm_w=dw, eps=1e-5, d=dd, x_out=xo, rope=rp)
        counts.append(len(plan))
        plan.destroy()
    assert counts[1] == counts[0] + (0 if folds else 1), counts
    for m, (y, mat, r) in enumerate(zip(ys, mats, rows)):
        want = oracle.matmul(t, mat, h, r)
        if m < n_rope:
            want = oracle.qk_norm_rope(want, n_tok, r // head_dim, head_dim, head_dim, pos, theta,
                                       mode).reshape(n_tok, r)
        assert rel_to_scale(y.numpy(), want) <= RTOL, f"matrix {m}"


def test_norm_matmul_rope_refusals(hip):
    """Refused before any launch: rows that are not whole heads, an odd head
    size, no positions, more rotated matrices than given."""
    import ctypes
    L = _lib.lib()
    n_cols, D = 1024, 64
    x = DA.empty((1, n_cols))
    m = DA.empty((96 * n_cols // 256 * 144,), np.uint8)
    y = DA.empty((1, 96))
    pos = DA.from_numpy(np.zeros(1, np.int32))
    inv = DA.from_numpy(np.ones(D // 2, np.float32))
    ws = DA.empty((1 << 20,), np.uint8)

    def call(rows, D, n_rope, pos_ptr):
        wp = (ctypes.c_void_p * 1)(m.ptr)
        wb = (ctypes.c_int64 * 1)(m.nbytes)
        nr = (ctypes.c_int64 * 1)(rows)
        yp = (ctypes.c_void_p * 1)(y.ptr)
        return L.aero_hip_norm_matmul_rope(W.Q4_K, 1, wp, wb, nr, yp, x.ptr, None, None, None,
                                           1e-5, 0, n_cols, 1, n_rope, D, 0, pos_ptr, inv.ptr,
                                           ws.ptr, ws.nbytes, None)
    assert call(96, 64, 1, pos.ptr) == 0 and "whole heads" in _lib.last_error()
    assert call(96, 33, 1, pos.ptr) == 0
    assert call(64, 64, 1, None) == 0
    assert call(64, 64, 2, pos.ptr) == 0
    assert call(64, 64, 1, pos.ptr) == 1


@pytest.mark.parametrize("t,n_cols,w_len", [(W.Q4_K, 1024, 128), (W.Q8_0, 512, 64),
                                             (W.Q6_K, 1024, 256)])
@pytest.mark.parametrize("n_tok", [1, 2, 3, 16, 40, 100])
def test_gated_norm_matmul_vs_oracle(hip, oracle, t, n_cols, w_len, n_tok):
    """The gated-DeltaNet norm folded into the projection after it, any token
    count: the fused GEMV's prologue (1-2 tokens), a gated norm pass then the
    GEMV (3-16; Q6_K rows of 840 bytes always), the split GEMM's x pre-pass
    (Q4_K from 16 tokens at this size), the fp32 GEMM on the normed rows (Q8_0
    from 32); against the oracle's gated_rmsnorm_silu then matmul."""
    rng = np.random.default_rng(n_cols + w_len + n_tok)
    n_rows = 512
    w = W.weight_table(t, n_rows, n_cols, rng)
    x = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    z = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(w_len)).astype(np.float32)
    y = DA.empty((n_tok, n_rows))
    print(f"gated_norm_matmul type={t} cols={n_cols} w_len={w_len} tokens={n_tok}", flush=True)
    ops.gated_norm_matmul(t, DA.from_numpy(w), DA.from_numpy(x), DA.from_numpy(z),
                          DA.from_numpy(nw), y, n_rows, n_cols, n_tok, 1e-6)
    want = oracle.matmul(t, w, oracle.gated_rmsnorm_silu(x, z, nw, 1e-6), n_rows)
    assert rel_to_scale(y.numpy(), want) <= RTOL
