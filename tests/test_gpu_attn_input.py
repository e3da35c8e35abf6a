"""GPU parity: aero_hip_attn_input, the attention sublayer's input in one call
(src/model.cpp:244-245,297-316; src/attention_layer.cpp:60-156): the residual
stream from the embedding rows or x + d, its RMSNorm, the projections sharing
it, then the per-head norm and RoPE of q and k -- against the oracle's
composition embed_gather -> rmsnorm_rows -> matmul -> qk_norm_rope.

With the split GEMM the embedding rows are dequantised in its x pre-pass and
the per-head norm and RoPE run in its epilogue when a workgroup's rows are
whole heads (head_dim 16-128): one pre-pass and one GEMM launch for every
step. Other paths (few tokens, heads of 256 rows, column splits) run the
gather + norm pass, the projections and the per-head pass. The residual
stream is bit-exact (the gather's dequant, or one IEEE add); the outputs are
within 1e-5 of their scale (the reference's RTOL,
tests/test_transformer_native.py:34-37)."""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import _lib, device, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA, Plan

pytestmark = pytest.mark.gpu

NEOX, INTER = ops.ROPE_NEOX, ops.ROPE_INTERLEAVED
THETA = 500000.0

CASES = [
    # (weights, table, tokens, columns, head_dim, heads (q, k, v[, gate]), n_rot, mode,
    #  qk norm, unit offset, x source, epilogue fold expected)
    (W.Q4_K, W.Q4_K, 64, 1024, 128, (8, 2, 2), 128, NEOX, False, False, "emb", True),
    (W.Q4_K, W.Q6_K, 64, 1024, 64, (8, 4, 4), 32, INTER, True, True, "emb", True),
    (W.Q8_0, W.Q8_0, 96, 2048, 128, (4, 1, 1, 4), 64, NEOX, True, False, "resid", True),
    (W.IQ4_XS, W.Q4_K, 40, 1024, 32, (8, 4, 4), 32, NEOX, False, False, "x", True),
    (W.Q5_K, W.Q8_0, 33, 1024, 16, (16, 8, 8), 16, INTER, True, False, "emb", True),
    (W.Q6_K, W.IQ4_XS, 64, 2048, 128, (4, 2, 2), 128, NEOX, False, False, "emb", True),
    # heads of 256 rows span two workgroups: the per-head pass follows
    (W.Q4_K, W.Q4_K, 64, 1024, 256, (4, 2, 2), 64, NEOX, True, False, "emb", False),
    # few tokens: gather + norm, the fused decode GEMV (RoPE in its epilogue
    # when every channel rotates and no head norm comes first)
    (W.Q4_K, W.Q4_K, 1, 1024, 128, (4, 2, 2), 128, NEOX, False, False, "emb", False),
    (W.Q4_K, W.Q5_K, 4, 1024, 64, (4, 2, 2), 64, INTER, True, True, "emb", False),
    (W.Q8_0, W.Q8_0, 2, 1024, 128, (4, 1, 1), 128, NEOX, False, False, "resid", False),
]


def table_for(t, vocab, n_cols, rng):
    return W.make_table(t, vocab * n_cols // W.BLOCK[t][0], rng)


def run_case(oracle, wt, et, T, N, D, heads, n_rot, mode, qk, uo, src, seed):
    rng = np.random.default_rng(seed)
    rows = [h * D for h in heads]
    vocab = 300
    table = table_for(et, vocab, N, rng)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    x = rng.standard_normal((T, N), dtype=np.float32)
    d = rng.standard_normal((T, N), dtype=np.float32)
    w = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.1) + 1).astype(np.float32)
    qw = (rng.standard_normal(D, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    kw = (rng.standard_normal(D, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    if not uo:
        qw, kw = qw + np.float32(1), kw + np.float32(1)
    mats = [W.make_table(wt, r * N // W.BLOCK[wt][0], rng) for r in rows]
    pos = rng.integers(0, 8192, T).astype(np.int32)
    n_rot, inv = ops.rope_inv_freq(D, n_rot, THETA)
    scale = float(np.float32(np.sqrt(N))) if et == W.Q6_K else 0.0
    print(f"attn_input w={wt} emb={et} T={T} N={N} D={D} heads={heads} n_rot={n_rot} "
          f"mode={mode} qk={qk} uo={uo} src={src}", flush=True)

    dmats = [DA.from_numpy(m) for m in mats]
    ys = [DA.empty((T, r)) for r in rows]
    xo = DA.empty((T, N))
    emb = ({"type": et, "table": DA.from_numpy(table), "vocab": vocab,
            "ids": DA.from_numpy(ids), "scale": scale} if src == "emb" else None)
    rope = {"n": 2, "head_dim": D, "n_rot": n_rot, "mode": mode, "pos": DA.from_numpy(pos),
            "inv_freq": DA.from_numpy(inv), "q_norm_w": DA.from_numpy(qw) if qk else None,
            "k_norm_w": DA.from_numpy(kw) if qk else None, "eps": 1e-6, "unit_offset": uo}
    dx = DA.from_numpy(x)
    dd = DA.from_numpy(d) if src == "resid" else None
    kw_args = dict(x_out=xo, x=None if src == "emb" else dx, d=dd, emb=emb,
                   norm_w=DA.from_numpy(w), eps=1e-5, rope=rope)
    ops.attn_input(wt, dmats, ys, rows, N, T, **kw_args)
    device.synchronize()

    if src == "emb":
        xs = oracle.embed_gather(et, table, vocab, N, ids, scale)
    elif src == "resid":
        xs = x + d
    else:
        xs = x
    if src != "x":
        assert bits_equal(xo.numpy(), xs), "residual stream"
    h = oracle.rmsnorm_rows(xs, w, 1e-5)
    for m, (y, mat, r) in enumerate(zip(ys, mats, rows)):
        want = oracle.matmul(wt, mat, h, r)
        if m < 2:
            want = oracle.qk_norm_rope(want, T, r // D, D, n_rot, pos, THETA, mode,
                                       (qw, kw)[m] if qk else None, 1e-6, uo).reshape(T, r)
        assert rel_to_scale(y.numpy(), want) <= RTOL, f"matrix {m}"
    return dmats, rows, kw_args, ys


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-T{c[2]}-D{c[4]}-{c[10]}")
def test_attn_input_vs_oracle(hip, oracle, case):
    wt, et, T, N, D, heads, n_rot, mode, qk, uo, src, fold = case
    # column splits (few workgroups) would move the per-head steps out of
    # the GEMM: one workgroup a row tile here, as at the model's shapes
    device.tune_set("gemm16_ksplit", 1)
    try:
        dmats, rows, kw_args, ys = run_case(oracle, wt, et, T, N, D, heads, n_rot, mode, qk, uo,
                                            src, seed=T * 13 + N + D + wt)
        plan = Plan()
        with plan:
            ops.attn_input(wt, dmats, [DA.empty(y.shape) for y in ys], rows, N, T, **kw_args)
        n = len(plan)
        plan.destroy()
    finally:
        device.tune_set("gemm16_ksplit", None)
    split = ops.split_ok(wt, N, sum(rows), T)
    if fold:
        assert split and n == 2, n     # pre-pass + GEMM
    elif split:
        assert n == 3, n               # pre-pass + GEMM + the per-head pass


@pytest.mark.parametrize("case", [c for c in CASES if c[11] and c[2] % 64 == 0 and c[0] in
                                  (W.Q4_K, W.Q6_K)],
                         ids=lambda c: f"{c[0]}-{c[1]}-T{c[2]}-D{c[4]}-{c[10]}")
def test_attn_input_64_token_workgroups(hip, oracle, case):
    """The per-head epilogue in 64-token workgroups (AERO_HIP_TUNE
    gemm16_mt=4; taken by itself when q/k/v has enough rows and tokens, e.g.
    2048 tokens at the Llama-3-8B shape): 16 channel pairs a thread, against
    the oracle; still one pre-pass and one GEMM launch."""
    wt, et, T, N, D, heads, n_rot, mode, qk, uo, src, fold = case
    device.tune_set("gemm16_ksplit", 1)
    device.tune_set("gemm16_mt", 4)
    try:
        dmats, rows, kw_args, ys = run_case(oracle, wt, et, T, N, D, heads, n_rot, mode, qk, uo,
                                            src, seed=T * 17 + N + D + wt)
        plan = Plan()
        with plan:
            ops.attn_input(wt, dmats, [DA.empty(y.shape) for y in ys], rows, N, T, **kw_args)
        n = len(plan)
        plan.destroy()
    finally:
        device.tune_set("gemm16_mt", None)
        device.tune_set("gemm16_ksplit", None)
    assert n == 2, n


def test_attn_input_llama3_8b_512_tokens(hip, oracle):
    """The Llama-3-8B block's attention input at 512 tokens (hidden 4096,
    32/8 heads of 128, Q4_K weights and table): two launches, checked on a
    sample of tokens across the token tiles."""
    rng = np.random.default_rng(8)
    T, N, D = 512, 4096, 128
    rows = [32 * D, 8 * D, 8 * D]
    vocab = 1000
    table = table_for(W.Q4_K, vocab, N, rng)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    w = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.1) + 1).astype(np.float32)
    mats = [W.weight_table(W.Q4_K, r, N, rng) for r in rows]
    pos = np.arange(T, dtype=np.int32)
    n_rot, inv = ops.rope_inv_freq(D, None, THETA)
    ys = [DA.empty((T, r)) for r in rows]
    xo = DA.empty((T, N))
    args = dict(x_out=xo, emb={"type": W.Q4_K, "table": DA.from_numpy(table), "vocab": vocab,
                               "ids": DA.from_numpy(ids)},
                norm_w=DA.from_numpy(w), eps=1e-5,
                rope={"n": 2, "head_dim": D, "mode": NEOX, "pos": DA.from_numpy(pos),
                      "inv_freq": DA.from_numpy(inv)})
    dmats = [DA.from_numpy(m) for m in mats]
    plan = Plan()
    with plan:
        ops.attn_input(W.Q4_K, dmats, ys, rows, N, T, **args)
    assert len(plan) == 2
    stream = device.Stream()
    plan.launch(stream)
    stream.synchronize()
    plan.destroy()
    xs = oracle.embed_gather(W.Q4_K, table, vocab, N, ids)
    assert bits_equal(xo.numpy(), xs)
    sample = np.array([0, 1, 31, 32, 100, 255, 256, 300, 511])
    h = oracle.rmsnorm_rows(xs[sample], w, 1e-5)
    for m, (y, mat, r) in enumerate(zip(ys, mats, rows)):
        want = oracle.matmul(W.Q4_K, mat, h, r)
        if m < 2:
            want = oracle.qk_norm_rope(want, sample.size, r // D, D, D, pos[sample], THETA,
                                       NEOX).reshape(sample.size, r)
        assert rel_to_scale(y.numpy()[sample], want) <= RTOL, f"matrix {m}"


def test_attn_input_bad_ids_give_zero_rows(hip, oracle):
    """An id outside the vocabulary gives a zero row of x (the gather's rule)
    and a zero h, so its q/k/v are zero; the other tokens are unaffected."""
    rng = np.random.default_rng(3)
    T, N, D, vocab = 64, 1024, 128, 50
    rows = [4 * D, 2 * D]
    table = table_for(W.Q4_K, vocab, N, rng)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    ids[[3, 40]] = [vocab, -1]
    mats = [W.make_table(W.Q4_K, r * N // 256, rng) for r in rows]
    n_rot, inv = ops.rope_inv_freq(D, None, THETA)
    ys = [DA.empty((T, r)) for r in rows]
    xo = DA.empty((T, N))
    ops.attn_input(W.Q4_K, [DA.from_numpy(m) for m in mats], ys, rows, N, T, x_out=xo,
                   emb={"type": W.Q4_K, "table": DA.from_numpy(table), "vocab": vocab,
                        "ids": DA.from_numpy(ids)},
                   rope={"n": 2, "head_dim": D, "pos": DA.from_numpy(np.arange(T, dtype=np.int32)),
                         "inv_freq": DA.from_numpy(inv)})
    device.synchronize()
    x = xo.numpy()
    assert not x[[3, 40]].any()
    good = np.setdiff1d(np.arange(T), [3, 40])
    assert bits_equal(x[good], oracle.embed_gather(W.Q4_K, table, vocab, N, ids[good]))
    for y in ys:
        assert not y.numpy()[[3, 40]].any()


def test_attn_input_refusals(hip):
    """Refused before any launch: a residual input with the embedding rows,
    rows that are not whole heads, an odd rotated width, no positions."""
    L = _lib.lib()
    N, T, D = 1024, 64, 128
    w = DA.from_numpy(np.zeros(D * N // 256 * 144, np.uint8))
    y = DA.empty((T, D))
    x = DA.empty((T, N))
    pos = DA.from_numpy(np.zeros(T, np.int32))
    inv = DA.from_numpy(np.ones(D // 2, np.float32))
    with pytest.raises(ValueError):
        ops.attn_input(W.Q4_K, [w], [y], [D], N, T, x_out=x, d=x,
                       emb={"type": W.Q4_K, "table": w, "vocab": 1, "ids": pos})

    import ctypes
    def call(rows, n_rot, p):
        a = _lib.AttnInput()
        wp = (ctypes.c_void_p * 1)(w.ptr)
        wb = (ctypes.c_int64 * 1)(w.nbytes)
        nr = (ctypes.c_int64 * 1)(rows)
        yp = (ctypes.c_void_p * 1)(y.ptr)
        a.dtype, a.n_mat, a.w, a.w_bytes, a.n_rows, a.y = W.Q4_K, 1, wp, wb, nr, yp
        a.n_cols, a.n_tok, a.x, a.x_out, a.norm = N, T, x.ptr, x.ptr, 0
        a.n_rope, a.head_dim, a.n_rot, a.pos, a.inv_freq = 1, D, n_rot, p, inv.ptr
        return L.aero_hip_attn_input(ctypes.byref(a), None, 0, None)

    assert call(D + 2, D, pos.ptr) == 0 and "whole heads" in _lib.last_error()
    assert call(D, D - 1, pos.ptr) == 0 and "RoPE" in _lib.last_error()
    assert call(D, D, None) == 0 and "RoPE" in _lib.last_error()
