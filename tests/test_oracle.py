"""CPU: pin the oracle (oracle/cpuref*.c) before trusting it to check the GPU path.

Every function is checked against at least one of: the reference's own C++
outputs (golden vectors from oracle/_ref, committed, and the live build when
present), the known-answer blocks of the reference's tests, float64 closed
forms, and the invariants the reference's tests assert. The last section
plants plausible mistakes in a numpy restatement and shows the same checks
reject them, so a check that passes is a check that could have failed.
"""
import math

import numpy as np
import pytest

from conftest import bits_equal, golden, rel_to_scale
from oracle import cpuref as O
from oracle import refbind as R

ref_built = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built here")


# ---------------------------------------------------------------- fp16 / quant
def test_f16_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(O.f16_bits_to_f32(h).view(np.uint32),
                          h.view(np.float16).astype(np.float32).view(np.uint32))


KATS = [("q4k_nibbles", O.Q4_K), ("q4k_pack_dmin0", O.Q4_K), ("q4k_pack_dmin1", O.Q4_K),
        ("q6k_zero", O.Q6_K), ("q6k_ones", O.Q6_K), ("q6k_lownib", O.Q6_K),
        ("q8_0_ramp", O.Q8_0)]


@pytest.mark.parametrize("name,t", KATS)
def test_quant_kat(name, t):
    k = golden("kat_quant.npz")
    want = k[name + "_want"]
    assert bits_equal(O.dequant(t, k[name + "_raw"], want.size), want)


def test_q4k_dmin_with_zero_mins_is_noop():
    k = golden("kat_quant.npz")
    assert bits_equal(O.dequant(O.Q4_K, k["q4k_nibbles_dmin2_raw"], 256), k["q4k_nibbles_want"])


def test_block_geometry():
    for t, bb, bv in ((O.Q8_0, 34, 32), (O.Q4_K, 144, 256), (O.Q6_K, 210, 256), (O.F16, 2, 1),
                      (O.F32, 4, 1), (O.BF16, 2, 1)):
        assert O.block_bytes(t) == bb and O.block_values(t) == bv


def test_dequant_refusals():
    with pytest.raises(ValueError):
        O.dequant(O.Q4_K, np.zeros(143, np.uint8), 256)      # short buffer
    with pytest.raises(ValueError):
        O.dequant(O.IQ4_XS, np.zeros(135, np.uint8), 256)    # short buffer
    with pytest.raises(ValueError):
        O.dequant(2, np.zeros(18, np.uint8), 32)             # Q4_0: no dequantiser
    assert O.dequant(O.Q8_0, np.zeros(34, np.uint8), 31).sum() == 0  # floor(n/bv) = 0 blocks


def test_threaded_dequant_bit_identical():
    rng = np.random.default_rng(3)
    from aero_amd import workloads as W
    for t in (O.Q8_0, O.Q4_K, O.Q6_K):
        raw = W.make_table(t, 333, rng)
        n = 333 * O.block_values(t)
        a = O.dequant(t, raw, n)
        for th in (2, 3, 8, 16):
            assert bits_equal(O.dequant(t, raw, n, threads=th), a)


# ---------------------------------------------------------------- golden vectors
def test_golden_norms_and_acts():
    g = golden("ref_vectors.npz")
    assert bits_equal(O.rmsnorm_rows(g["norm_x"], g["norm_w"], 1e-6), g["rms_out"])
    assert bits_equal(O.rmsnorm_rows(g["norm_x"], None, 1e-6), g["rms_out_noweight"])
    assert bits_equal(O.l2norm_rows(g["norm_x"], g["norm_w"], 1e-6), g["l2_out"])
    assert bits_equal(O.rmsnorm_rows(g["rms4096_x"], g["rms4096_w"], 1e-5), g["rms4096_out"])
    z, up = g["act_z"], g["act_up"]
    assert bits_equal(O.act(O.ACT_SILU, z), g["silu_out"])
    assert bits_equal(O.act(O.ACT_GELU, z), g["gelu_out"])
    assert bits_equal(O.act_mul(O.ACT_SILU, z, up), g["swiglu_out"])
    assert bits_equal(O.act_mul(O.ACT_IDENTITY, z, up), g["mul_out"])


def test_golden_rope():
    g = golden("ref_vectors.npz")
    pos = g["rope_pos"]
    ff = np.concatenate([np.ones(16, np.float32), np.full(16, 1e30, np.float32)])
    for tag, hd, nd, base, f in (("full128", 128, None, 500000.0, None),
                                 ("partial64of256", 256, 64, 1e7, None),
                                 ("ff64", 64, None, 10000.0, ff)):
        c, s = O.rope_tables(hd, pos, base, nd, f)
        assert bits_equal(c, g[f"tab_{tag}_cos"]) and bits_equal(s, g[f"tab_{tag}_sin"]), tag
    x, c, s, rp = g["apply_x"], g["apply_cos"], g["apply_sin"], g["apply_pos"]
    assert bits_equal(O.apply_rope(x, c, s, rp, 0), g["apply_neox"])
    assert bits_equal(O.apply_rope(x, c, s, rp, 1), g["apply_inter"])
    assert bits_equal(O.apply_rope(x, g["apply_cos8"], g["apply_sin8"], rp, 0),
                      g["apply_partial8"])


def test_golden_dequant():
    g = golden("ref_vectors.npz")
    for t in (8, 12, 13, 14, 23):
        want = g[f"deq{t}_out"]
        assert bits_equal(O.dequant(t, g[f"deq{t}_raw"], want.size), want)


def scale_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_golden_matvec_matmul():
    """The reference's own matvec / matmul outputs (src/kernels.cpp:497-538).
    The reference is built with -ffast-math, so its sums may be reassociated:
    within 1e-6 of the output scale (bit-exact for four of the five types)."""
    g = golden("ref_vectors.npz")
    for t in (8, 12, 13, 14, 23):
        w, X = g[f"mv{t}_w"], g[f"mv{t}_x"]
        n_rows = g[f"mv{t}_y"].size
        y = O.matvec(t, w, X[0], n_rows)
        assert scale_err(y, g[f"mv{t}_y"]) <= 1e-6, t
        Y = O.matmul(t, w, X, n_rows)
        assert scale_err(Y, g[f"mm{t}_y"]) <= 1e-6, t
        # every token row of matmul is that token's matvec (tests/test_kernels.cpp:289-314)
        for i in range(X.shape[0]):
            assert bits_equal(Y[i], O.matvec(t, w, X[i], n_rows))


# ------------------------------------------------------ live reference build
@ref_built
def test_live_reference_fp32_path():
    rng = np.random.default_rng(99)
    for rows, cols in ((1, 1), (3, 7), (17, 896), (5, 4096), (2, 8193)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        w = rng.standard_normal(cols).astype(np.float32)
        assert bits_equal(O.rmsnorm_rows(x, w, 1e-5), R.rmsnorm_rows(x, w, 1e-5))
        assert bits_equal(O.l2norm_rows(x, None, 1e-6), R.l2norm_rows(x, None, 1e-6))
    z = (rng.standard_normal(9999) * 6).astype(np.float32)
    u = rng.standard_normal(9999).astype(np.float32)
    assert bits_equal(O.act(0, z), R.act("silu", z))
    assert bits_equal(O.act(1, z), R.act("gelu", z))
    assert bits_equal(O.act_mul(0, z, u), R.swiglu(z, u))
    for hd, nd, base in ((128, None, 5e5), (256, 64, 1e7), (64, None, 1e6), (80, 48, 1e4)):
        pos = rng.integers(0, 65536, 50).astype(np.int32)
        a, b = O.rope_tables(hd, pos, base, nd), R.rope_tables(hd, pos, base, nd)
        assert bits_equal(a[0], b[0]) and bits_equal(a[1], b[1])
        xr = rng.standard_normal((50, hd)).astype(np.float32)
        rows = np.arange(50, dtype=np.int32)
        for mode in (0, 1):
            assert bits_equal(O.apply_rope(xr, a[0], a[1], rows, mode),
                              R.apply_rope(xr, a[0], a[1], rows, mode))


@ref_built
def test_live_reference_dequant():
    from aero_amd import workloads as W
    rng = np.random.default_rng(98)
    for t in (O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_XS):
        raw = W.make_table(t, 257, rng)
        n = 257 * O.block_values(t)
        assert bits_equal(O.dequant(t, raw, n), R.dequant(t, raw, n))
    raw = rng.integers(0, 256, 2000, dtype=np.uint8)
    for t in (O.F16, O.BF16, O.F32):
        n = 2000 // O.block_bytes(t)
        a, b = O.dequant(t, raw, n), R.dequant(t, raw, n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@ref_built
def test_live_reference_matvec():
    from aero_amd import workloads as W
    rng = np.random.default_rng(97)
    for t in (O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_XS):
        bv = O.block_values(t)
        for n_rows, n_cols in ((1, bv), (37, 4 * 256), (5, 4096)):
            w = W.make_table(t, n_rows * n_cols // bv, rng)
            X = rng.standard_normal((2, n_cols)).astype(np.float32)
            assert scale_err(O.matvec(t, w, X[0], n_rows), R.matvec(t, w, X[0], n_rows)) <= 1e-6
            assert scale_err(O.matmul(t, w, X, n_rows), R.matmul(t, w, X, n_rows)) <= 1e-6


def test_q5k_iq4xs_closed_forms():
    """Q5_K with qh = 0 is Q4_K of the same fields; each qh bit adds 16 to its
    quant; IQ4_XS with one nibble value per block is dl * codebook[value]."""
    from aero_amd import workloads as W
    rng = np.random.default_rng(96)
    q4 = W.make_table(O.Q4_K, 8, rng).reshape(8, 144)
    q5 = np.zeros((8, 176), np.uint8)
    q5[:, :16], q5[:, 48:] = q4[:, :16], q4[:, 16:]
    assert bits_equal(O.dequant(O.Q5_K, q5, 8 * 256), O.dequant(O.Q4_K, q4, 8 * 256))
    q5[:, 16:48] = 0xFF
    d = _f16(q5[:, 0:2].copy()).astype(np.float64).reshape(-1, 1)
    dmin = _f16(q5[:, 2:4].copy()).astype(np.float64).reshape(-1, 1)
    got = O.dequant(O.Q5_K, q5, 8 * 256).reshape(8, 256).astype(np.float64)
    base = O.dequant(O.Q4_K, q4, 8 * 256).reshape(8, 256).astype(np.float64)
    # every value gains 16 * d * sc of its sub-block: (got - base) / d is 16*sc, an integer
    steps = (got - base) / d
    assert np.allclose(steps, np.round(steps), atol=1e-3) and (np.round(steps) % 16 == 0).all()
    del dmin
    codebook = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89,
                         113], np.float32)
    for k in range(16):
        blk = np.zeros(136, np.uint8)
        blk[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
        blk[2:4] = [0b10010011, 0b01101100]           # scales_h: 2 bits per sub-block
        blk[4:8] = [0x21, 0x43, 0x65, 0x87]           # scales_l: 4 bits per sub-block
        blk[8:] = k | (k << 4)
        out = O.dequant(O.IQ4_XS, blk, 256).reshape(8, 32)
        sh = int(blk[2]) | (int(blk[3]) << 8)
        for ib in range(8):
            ls = ((int(blk[4 + ib // 2]) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
            dl = np.float32(0.25) * np.float32(ls - 32)
            assert bits_equal(out[ib], np.full(32, dl * codebook[k], np.float32)), (k, ib)


def test_matvec_is_dequant_times_x():
    """y = dequant(W) @ x, evaluated in float64 (the definition of matvec)."""
    from aero_amd import workloads as W
    rng = np.random.default_rng(95)
    for t in (O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ4_XS):
        n_rows, n_cols = 19, 2048
        bv = O.block_values(t)
        w = W.make_table(t, n_rows * n_cols // bv, rng)
        x = rng.standard_normal(n_cols).astype(np.float32)
        Wf = O.dequant(t, w, n_rows * n_cols).astype(np.float64).reshape(n_rows, n_cols)
        assert scale_err(O.matvec(t, w, x, n_rows), Wf @ x.astype(np.float64)) <= 1e-6, t
    with pytest.raises(ValueError):
        O.matvec(O.Q4_K, np.zeros(144, np.uint8), np.zeros(255, np.float32), 1)   # n_cols % 256
    with pytest.raises(ValueError):
        O.matvec(O.F32, np.zeros(64, np.uint8), np.zeros(16, np.float32), 1)     # not a block type


# ------------------------------------------------------------- closed forms
def test_rmsnorm_closed_form():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((9, 2560)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2560)).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert rel_to_scale(O.rmsnorm_rows(x, w, 1e-6), want) < 1e-6
    # Gemma (1+w) is the composition with w' = 1 + w in fp32
    assert bits_equal(O.rmsnorm_rows(x, w - 1, 1e-6, unit_offset=True),
                      O.rmsnorm_rows(x, np.float32(1) + (w - np.float32(1)), 1e-6))
    # weight None == ones, bit for bit; ones in -> weight out
    assert bits_equal(O.rmsnorm_rows(x, None, 1e-6), O.rmsnorm_rows(x, np.ones(2560, np.float32), 1e-6))
    assert np.allclose(O.rmsnorm_rows(np.ones((2, 2560), np.float32), w, 1e-6), w, rtol=1e-5)


def test_l2norm_closed_form_and_floor():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.maximum(np.linalg.norm(x64, axis=1, keepdims=True), 1e-6)
    assert rel_to_scale(O.l2norm_rows(x, None, 1e-6), want) < 1e-6
    tiny = np.full((1, 64), 1e-9, np.float32)
    got = np.linalg.norm(O.l2norm_rows(tiny, None, 1e-6).astype(np.float64))
    assert abs(got - 8e-9 / 1e-6) / (8e-9 / 1e-6) < 1e-3


def test_gated_norm_closed_form_and_invariants():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 4096)).astype(np.float32)
    z = rng.standard_normal((6, 4096)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    x64, z64 = x.astype(np.float64), z.astype(np.float64)
    for group in (4096, 128):
        xg = x64.reshape(6, -1, group)
        nrm = xg / np.sqrt((xg ** 2).mean(axis=2, keepdims=True) + 1e-6)
        want = nrm.reshape(6, 4096) * np.tile(w, 32) * (z64 / (1 + np.exp(-z64)))
        assert rel_to_scale(O.gated_rmsnorm_silu(x, z, w, 1e-6, group), want) < 1e-6
    big = np.full_like(z, 60.0)
    out = O.gated_rmsnorm_silu(x, big, np.ones(128, np.float32), 1e-6).astype(np.float64) / 60
    assert np.allclose(np.sqrt((out ** 2).mean(axis=1)), 1.0, atol=1e-5)


def test_activation_closed_forms():
    z = np.linspace(-8, 8, 4001, dtype=np.float32)
    z64 = z.astype(np.float64)
    gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in z64])
    tanh = 0.5 * z64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (z64 + 0.044715 * z64 ** 3)))
    assert np.abs(O.act(O.ACT_GELU, z) - gelu).max() < 2e-6
    assert rel_to_scale(O.act(O.ACT_GELU_TANH, z), tanh) < 1e-6
    assert rel_to_scale(O.act(O.ACT_SILU, z), z64 / (1 + np.exp(-z64))) < 1e-6
    # the erf form is not the tanh form (tests/test_tensor_native.py:118-126)
    assert np.abs(O.act(O.ACT_GELU, z) - tanh).max() > 1e-4


def test_rope_closed_form():
    pos = np.array([0, 1, 37, 511, 4095, 16383, 32767], np.int32)
    for hd, nd, base in ((128, None, 5e5), (256, 64, 1e7)):
        n, inv = O.rope_inv_freq(hd, nd, base)
        inv64 = 1.0 / (np.float64(base) ** (np.arange(n // 2) * 2.0 / n))
        assert np.abs(inv / inv64 - 1).max() < 1e-6
        c, s = O.rope_tables(hd, pos, base, nd)
        ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)  # fp32 angle
        assert np.abs(c - np.cos(ang)).max() < 1e-6 and np.abs(s - np.sin(ang)).max() < 1e-6
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    c, s = O.rope_tables(64, np.arange(5), 1e4)
    rows = np.arange(5, dtype=np.int32)
    x64, c64, s64 = x.astype(np.float64), c.astype(np.float64), s.astype(np.float64)
    want = x64.copy()
    want[:, :32] = x64[:, :32] * c64 - x64[:, 32:] * s64
    want[:, 32:] = x64[:, :32] * s64 + x64[:, 32:] * c64
    assert rel_to_scale(O.apply_rope(x, c, s, rows, 0), want) < 1e-6


def test_rope_properties():
    rng = np.random.default_rng(9)
    D = 16
    q0, k0 = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    c, s = O.rope_tables(D, np.arange(32), 1e4)

    def score(qp, kp, mode):
        q = O.apply_rope(q0[None], c, s, np.array([qp], np.int32), mode)[0]
        k = O.apply_rope(k0[None], c, s, np.array([kp], np.int32), mode)[0]
        return float(np.dot(q.astype(np.float64), k))

    for mode in (0, 1):
        base = score(0, 5, mode)
        assert max(abs(score(t, t + 5, mode) - base) for t in range(1, 21)) < 1e-4
        assert abs(score(5, 0, mode) - base) > 1e-3   # not symmetric
        r = O.apply_rope(q0[None], c, s, np.array([7], np.int32), mode)[0]
        assert abs(np.linalg.norm(r) - np.linalg.norm(q0)) < 1e-5
    c8, s8 = O.rope_tables(D, np.arange(32), 1e4, 8)
    r = O.apply_rope(q0[None], c8, s8, np.array([5], np.int32), 0)[0]
    assert bits_equal(r[8:], q0[8:]) and not np.allclose(r[:8], q0[:8])
    ff = np.concatenate([np.ones(4, np.float32), np.full(4, 1e30, np.float32)])
    cf, sf = O.rope_tables(D, np.arange(1, 6), 1e4, None, ff)
    # tests/test_transformer_cpp.cpp:137-158: cos -> 1, sin -> 0 within 1e-5
    assert np.abs(cf[:, 4:] - 1).max() < 1e-5 and np.abs(sf[:, 4:]).max() < 1e-5
    with pytest.raises(ValueError):
        O.rope_tables(D, np.arange(3), 1e4, None, np.ones(3, np.float32))


def test_embed_gather_rows_and_refusals():
    from aero_amd import workloads as W
    rng = np.random.default_rng(10)
    for t in (O.Q8_0, O.Q4_K, O.Q6_K):
        bv, bb = W.BLOCK[t]
        table = W.make_table(t, 40 * 2, rng)
        ids = rng.integers(0, 40, 25).astype(np.int32)
        got = O.embed_gather(t, table, 40, 2 * bv, ids)
        for i, tok in enumerate(ids):
            assert bits_equal(got[i], O.dequant(t, table[tok * 2 * bb:(tok + 1) * 2 * bb], 2 * bv))
        scaled = O.embed_gather(t, table, 40, 2 * bv, ids, scale=float(np.float32(math.sqrt(2560))))
        assert bits_equal(scaled, got * np.float32(math.sqrt(2560)))
        with pytest.raises(ValueError):
            O.embed_gather(t, table, 40, 2 * bv, np.array([40], np.int32))
        with pytest.raises(ValueError):
            O.embed_gather(t, table, 40, 2 * bv, np.array([-1], np.int32))
        with pytest.raises(ValueError):
            O.embed_gather(t, table, 40, bv + 1, ids)


# ------------------------------------------------------------ planted mistakes
def _f16(b):
    return b.view(np.float16).astype(np.float32)


def np_q4k(raw, swap_nibbles=False, naive_scales=False):
    """numpy restatement of Q4_K with optional planted mistakes."""
    a = raw.reshape(-1, 144)
    d, dmin = _f16(a[:, 0:2].copy()).reshape(-1), _f16(a[:, 2:4].copy()).reshape(-1)
    sc, qs = a[:, 4:16].astype(np.int32), a[:, 16:].astype(np.int32)
    out = np.empty((a.shape[0], 256), np.float32)

    def sm(k):
        if k < 4 or naive_scales:
            return sc[:, k % 8] & 63, sc[:, (k + 4) % 12] & 63
        return (sc[:, k + 4] & 15) | ((sc[:, k - 4] >> 6) << 4), (sc[:, k + 4] >> 4) | ((sc[:, k] >> 6) << 4)

    for j in range(4):
        s1, m1 = sm(2 * j)
        s2, m2 = sm(2 * j + 1)
        lo, hi = qs[:, 32 * j:32 * j + 32] & 15, qs[:, 32 * j:32 * j + 32] >> 4
        if swap_nibbles:
            lo, hi = hi, lo
        out[:, 64 * j:64 * j + 32] = (d * s1.astype(np.float32))[:, None] * lo - (dmin * m1.astype(np.float32))[:, None]
        out[:, 64 * j + 32:64 * j + 64] = (d * s2.astype(np.float32))[:, None] * hi - (dmin * m2.astype(np.float32))[:, None]
    return out.reshape(-1)


def np_q6k(raw, qh_shift_off=0):
    a = raw.reshape(-1, 210)
    ql, qh = a[:, :128].astype(np.int32), a[:, 128:192].astype(np.int32)
    sc = a[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16(a[:, 208:210].copy()).reshape(-1)
    out = np.empty((a.shape[0], 256), np.float32)
    for h in range(2):
        for l in range(32):
            lo, hi, hb = ql[:, 64 * h + l], ql[:, 64 * h + l + 32], qh[:, 32 * h + l]
            qv = [(lo & 15) | (((hb >> (0 + qh_shift_off)) & 3) << 4),
                  (hi & 15) | (((hb >> (2 + qh_shift_off)) & 3) << 4),
                  (lo >> 4) | (((hb >> 4) & 3) << 4), (hi >> 4) | (((hb >> 6) & 3) << 4)]
            for k in range(4):
                out[:, 128 * h + l + 32 * k] = d * sc[:, 8 * h + l // 16 + 2 * k] * (qv[k] - 32).astype(np.float32)
    return out.reshape(-1)


def np_iq4xs(raw, swap_scale_bits=False):
    """numpy restatement of IQ4_XS dequant, with an optional planted mistake."""
    cb = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                  np.float32)
    a = raw.reshape(-1, 136)
    d = _f16(a[:, 0:2].copy()).reshape(-1)
    sh = a[:, 2].astype(np.int32) | (a[:, 3].astype(np.int32) << 8)
    out = np.empty((a.shape[0], 256), np.float32)
    for ib in range(8):
        lo = (a[:, 4 + ib // 2].astype(np.int32) >> (4 * (ib % 2))) & 15
        hi = (sh >> (2 * (7 - ib if swap_scale_bits else ib))) & 3
        dl = d * ((lo | (hi << 4)) - 32).astype(np.float32)
        q = a[:, 8 + 16 * ib:8 + 16 * ib + 16]
        out[:, 32 * ib:32 * ib + 16] = dl[:, None] * cb[q & 15]
        out[:, 32 * ib + 16:32 * ib + 32] = dl[:, None] * cb[q >> 4]
    return out.reshape(-1)


def np_matvec_q4k(w, x, n_rows, drop_min=False):
    """numpy Q4_K matvec through dequant, optionally dropping the dmin*m term."""
    a = w.reshape(n_rows, -1, 144)
    y = np.zeros(n_rows)
    for r in range(n_rows):
        for b in range(a.shape[1]):
            blk = a[r, b].copy()
            if drop_min:
                blk[2:4] = 0
            y[r] += O.dequant(O.Q4_K, blk, 256).astype(np.float64) @ x[256 * b:256 * (b + 1)]
    return y


def test_planted_quant_mistakes_are_caught():
    k = golden("kat_quant.npz")
    g = golden("ref_vectors.npz")
    raw = k["q4k_pack_dmin1_raw"]
    want = k["q4k_pack_dmin1_want"]
    assert bits_equal(np_q4k(raw), want)                      # the restatement passes
    assert not bits_equal(np_q4k(raw, swap_nibbles=True), want)
    assert not bits_equal(np_q4k(g["deq12_raw"], naive_scales=True), g["deq12_out"])
    assert bits_equal(np_q6k(g["deq14_raw"]), g["deq14_out"])
    assert not bits_equal(np_q6k(g["deq14_raw"], qh_shift_off=1), g["deq14_out"])
    assert bits_equal(np_iq4xs(g["deq23_raw"]), g["deq23_out"])
    assert not bits_equal(np_iq4xs(g["deq23_raw"], swap_scale_bits=True), g["deq23_out"])
    w, x = g["mv12_w"], g["mv12_x"][0].astype(np.float64)
    n_rows = g["mv12_y"].size
    assert scale_err(np_matvec_q4k(w, x, n_rows), g["mv12_y"]) <= 1e-6
    assert scale_err(np_matvec_q4k(w, x, n_rows, drop_min=True), g["mv12_y"]) > 1e-3


def test_planted_fp32_mistakes_are_caught():
    g = golden("ref_vectors.npz")
    x, w = g["norm_x"].astype(np.float64), g["norm_w"].astype(np.float64)
    sum_not_mean = x / np.sqrt((x ** 2).sum(axis=1, keepdims=True) + 1e-6) * w
    assert rel_to_scale(sum_not_mean, g["rms_out"]) > 1e-2
    xr, c, s, rp = g["apply_x"], g["apply_cos"], g["apply_sin"], g["apply_pos"]
    # NeoX read with interleaved pairing (the wrong mode) is rejected
    assert not bits_equal(O.apply_rope(xr, c, s, rp, 1), g["apply_neox"])
    # partial rotary with the head_dim exponent instead of n_rot's (F5) is rejected
    pos = g["rope_pos"]
    c_wrong = np.cos(pos.astype(np.float64)[:, None] /
                     (1e7 ** (np.arange(32) * 2.0 / 256)))
    assert np.abs(c_wrong - g["tab_partial64of256_cos"]).max() > 1e-2
    # tanh GELU where the erf form is required is rejected
    z = g["act_z"].astype(np.float64)
    tanh = 0.5 * z * (1 + np.tanh(math.sqrt(2 / math.pi) * (z + 0.044715 * z ** 3)))
    assert np.abs(tanh - g["gelu_out"]).max() > 1e-4


# ------------------------------------------------------ softmax / attention
def _attn_f64(q, k, v, scale, qpos=None, kpos=None, window=None):
    """Definition of the reference's attention in float64: per (token, head),
    softmax over the kept keys of (q . k) * scale, times v; zero when no key is
    kept. GQA: head h reads kv head h // (H // HK)."""
    T, H, D = q.shape
    S, HK, DV = k.shape[0], k.shape[1], v.shape[2]
    rep = H // HK
    qp = np.arange(T) if qpos is None else np.asarray(qpos)
    kp = np.arange(S) if kpos is None else np.asarray(kpos)
    out = np.zeros((T, H, DV))
    for t in range(T):
        keep = kp <= qp[t]
        if window:
            keep &= (qp[t] - kp) < window
        if not keep.any():
            continue
        for h in range(H):
            s = (k[keep, h // rep].astype(np.float64) @ q[t, h].astype(np.float64)) * scale
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[keep, h // rep].astype(np.float64)
    return out


def test_golden_softmax_attention_kv():
    """The reference's own softmax, attention and KV quantiser outputs."""
    g = golden("ref_vectors.npz")
    assert bits_equal(O.softmax(g["softmax_x"]), g["softmax_y"])
    q, k, v, qpos = g["att_q"], g["att_k"], g["att_v"], g["att_qpos"]
    assert bits_equal(O.attention_tiled(q, k, v, 0.125, qpos=qpos, block=16), g["att_out"])
    assert bits_equal(O.attention_tiled(q, k, v, 0.125, qpos=qpos, block=16, window=8),
                      g["att_out_win8"])
    assert bits_equal(O.attention_tiled(q, k, v, 0.125, qpos=qpos, kpos=g["att_kpos"]),
                      g["att_out_kpos"])
    for dt in (1, 2):
        for i, row in enumerate(g["kv_x"]):
            qb, sc = O.kv_write_vec(dt, row)
            assert np.array_equal(qb, g[f"kv{dt}_q"][i]) and np.float32(sc) == g[f"kv{dt}_scale"][i]


def test_live_reference_attention():
    """Bit-identical to the compiled reference (src/transformer.cpp) across
    GQA ratios, block sizes, windows, positions and the decode entry."""
    if R.transformer() is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(41)
    for (T, H, HK, D, DV, S) in ((1, 32, 8, 128, 128, 300), (9, 6, 6, 16, 24, 40),
                                 (4, 4, 1, 32, 32, 70)):
        q = rng.standard_normal((T, H, D)).astype(np.float32)
        k = rng.standard_normal((S, HK, D)).astype(np.float32)
        v = rng.standard_normal((S, HK, DV)).astype(np.float32)
        qpos = rng.integers(-1, S + 2, T).astype(np.int32)
        kpos = rng.permutation(S).astype(np.int32)
        for block, window, kp in ((1024, None, None), (13, None, None), (32, 9, None),
                                  (64, None, kpos)):
            a = O.attention_tiled(q, k, v, 0.1, qpos=qpos, kpos=kp, block=block, window=window)
            b = R.attention_tiled(q, k, v, 0.1, qpos=qpos, kpos=kp, block=block, window=window)
            assert bits_equal(a, b)
    x = (rng.standard_normal((5, 1000)) * 10).astype(np.float32)
    assert bits_equal(O.softmax(x), R.softmax(x))
    if R.kv() is not None:
        for dt in (0, 1, 2):
            xv = (rng.standard_normal(128) * 5).astype(np.float32)
            qa, sa = O.kv_write_vec(dt, xv)
            qb, sb = R.kv_write_vec(dt, xv)
            assert np.array_equal(qa, qb) and sa == sb
            assert bits_equal(O.kv_read_vec(dt, qa, sa, 128), R.kv_read_vec(dt, qb, sb, 128))


def test_attention_definition_and_invariants():
    """Against the float64 definition (masked softmax times V, GQA by integer
    division of the head), plus: a fully masked query gives exactly zero, one
    kept key returns its value row, the block size changes only rounding, and
    a planted head mapping (h % HK) is rejected."""
    rng = np.random.default_rng(43)
    T, H, HK, D, DV, S = 6, 8, 2, 16, 20, 33
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((S, HK, D)).astype(np.float32)
    v = rng.standard_normal((S, HK, DV)).astype(np.float32)
    qpos = np.array([0, 3, 10, 32, 32, -5], np.int32)
    for window in (None, 4):
        got = O.attention_tiled(q, k, v, 0.3, qpos=qpos, block=7, window=window)
        want = _attn_f64(q, k, v, 0.3, qpos=qpos, window=window)
        assert rel_to_scale(got, want) <= 1e-6
    got = O.attention_tiled(q, k, v, 0.3, qpos=qpos)
    assert not got[5].any()                                          # position -5: nothing kept
    for h in range(H):                                               # position 0: key 0 only
        assert bits_equal(got[0, h], v[0, h // (H // HK)])
    a = O.attention_tiled(q, k, v, 0.3, qpos=qpos, block=5)
    b = O.attention_tiled(q, k, v, 0.3, qpos=qpos, block=1024)
    assert rel_to_scale(a, b) <= 1e-6
    # a planted mistake: kv head h % HK instead of h // rep
    bad = np.zeros((T, H, DV))
    for h in range(H):
        bad[:, h] = _attn_f64(q[:, [h]], k[:, [h % HK]], v[:, [h % HK]], 0.3, qpos=qpos)[:, 0]
    assert rel_to_scale(O.attention_tiled(q, k, v, 0.3, qpos=qpos), bad) > 1e-3
    # decode entry = one query at position S-1
    dq = rng.standard_normal((H, D)).astype(np.float32)
    assert bits_equal(O.attention(dq, k, v, 0.3),
                      O.attention_tiled(dq[None], k, v, 0.3, qpos=[S - 1], block=S)[0])


def test_softmax_and_kv_closed_forms():
    """softmax rows sum to 1 and equal the float64 definition; int8 / int4
    quantisation: scale = amax/127 (amax/7), 1 for a zero vector, every value
    within scale/2 of x, int4 low nibble first and sign-extended on read."""
    rng = np.random.default_rng(47)
    x = (rng.standard_normal((4, 50)) * 6).astype(np.float32)
    y = O.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert np.allclose(y, e / e.sum(1, keepdims=True), rtol=1e-6, atol=1e-7)
    for dt, qmax in ((1, 127), (2, 7)):
        xv = (rng.standard_normal(64) * 3).astype(np.float32)
        qb, sc = O.kv_write_vec(dt, xv)
        assert np.float32(sc) == np.float32(np.abs(xv).max()) / np.float32(qmax)
        back = O.kv_read_vec(dt, qb, sc, 64)
        assert np.all(np.abs(back.astype(np.float64) - xv) <= sc / 2 * (1 + 1e-6))
        z = O.kv_write_vec(dt, np.zeros(64, np.float32))
        assert z[1] == 1.0 and not z[0].any()
    qb, sc = O.kv_write_vec(2, np.array([1.0, -7.0] + [0.0] * 6, np.float32))
    assert sc == 1.0 and qb[0] == (1 | (0x9 << 4))                  # -7 & 15 = 9, high nibble
    assert list(O.kv_read_vec(2, qb, sc, 8)[:2]) == [1.0, -7.0]


# ------------------------------------------------------------ gated DeltaNet

def _ssm_inputs(rng, T, n_k, n_v, d):
    q = rng.standard_normal((T, n_k, d)).astype(np.float32)
    k = rng.standard_normal((T, n_k, d)).astype(np.float32)
    v = rng.standard_normal((T, n_v, d)).astype(np.float32)
    alpha = rng.standard_normal((T, n_v)).astype(np.float32)
    beta = rng.standard_normal((T, n_v)).astype(np.float32)
    a_log = (-np.abs(rng.standard_normal(n_v)) * 0.5).astype(np.float32)
    dt_bias = rng.standard_normal(n_v).astype(np.float32)
    state = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
    return q, k, v, alpha, beta, a_log, dt_bias, state


def _ssm_f64_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """The gated delta rule in float64 from its definition (engine/ssm.py:1-20
    recurrence; v-head h reads k-head h % n_k)."""
    n_k, d = q.shape
    n_v = v.shape[0]
    S = state.astype(np.float64).copy()
    out = np.zeros((n_v, d))
    for h in range(n_v):
        qn = q[h % n_k].astype(np.float64)
        kn = k[h % n_k].astype(np.float64)
        qn /= max(np.linalg.norm(qn), eps)
        kn /= max(np.linalg.norm(kn), eps)
        x = float(alpha[h]) + float(dt_bias[h])
        g = min(float(a_log[h]) * (np.log1p(np.exp(-abs(x))) + max(x, 0.0)), 0.0)
        b = 1.0 / (1.0 + np.exp(-float(beta[h])))
        S[h] *= np.exp(g)
        S[h] += np.outer(kn, (v[h] - kn @ S[h]) * b)
        out[h] = scale * (qn @ S[h])
    return out, S


def test_ssm_matches_compiled_reference():
    """Bit-identical to src/ssm.cpp built into oracle/_ref: softplus over
    [-30, 30], the delta step (tiled heads), the grouped scan and the conv
    with its tail, over two chunks."""
    if R.ssm() is None:
        pytest.skip("oracle/_ref not built")
    L = R.ssm()
    xs = np.linspace(-30, 30, 401).astype(np.float32)
    assert bits_equal(O.ssm_softplus(xs), np.array([L.aero_ssm_softplus(float(x)) for x in xs],
                                                   np.float32))
    rng = np.random.default_rng(51)
    q, k, v, al, bt, a_log, dt, st = _ssm_inputs(rng, 5, 2, 4, 16)
    qe, ke = np.tile(q[0], (2, 1)), np.tile(k[0], (2, 1))
    o1, s1 = O.ssm_delta_step(qe, ke, v[0], al[0], bt[0], a_log, dt, st, 0.25)
    o2, s2 = R.ssm_delta_step(qe, ke, v[0], al[0], bt[0], a_log, dt, st, 0.25)
    assert bits_equal(o1, o2) and bits_equal(s1, s2)
    o1, s1 = O.ssm_scan(q, k, v, al, bt, a_log, dt, st, 0.25)
    o2, s2 = R.ssm_scan(q, k, v, al, bt, a_log, dt, st, 0.25)
    assert bits_equal(o1, o2) and bits_equal(s1, s2)
    x = rng.standard_normal((7, 10)).astype(np.float32)
    w = rng.standard_normal((10, 4)).astype(np.float32)
    t0 = np.zeros((3, 10), np.float32)
    for a, b in ((0, 2), (2, 7)):
        r1 = O.ssm_conv(x[a:b], w, t0, 0 if a == 0 else tl)
        r2 = R.ssm_conv(x[a:b], w, t0, 0 if a == 0 else tl)
        assert bits_equal(r1[0], r2[0]) and r1[2] == r2[2]
        assert bits_equal(r1[1][:r1[2]], r2[1][:r2[2]])
        t0, tl = r1[1], r1[2]


def test_ssm_definition_and_invariants():
    """Against the float64 definition; the delta rule's closed form (no decay,
    beta -> 1: the written key reads back its value, kn^T S' = v); beta -> 0
    leaves the decayed state; the conv in two chunks equals one pass; planted
    mistakes (h // ratio grouping, reversed conv taps) are rejected."""
    rng = np.random.default_rng(53)
    q, k, v, al, bt, a_log, dt, st = _ssm_inputs(rng, 3, 2, 6, 12)
    out, S = O.ssm_delta_step(q[0], k[0], v[0], al[0], bt[0], a_log, dt, st, 0.3)
    want, Sw = _ssm_f64_step(q[0], k[0], v[0], al[0], bt[0], a_log, dt, st, 0.3)
    assert np.abs(out - want).max() <= 1e-5 * np.abs(want).max()
    assert np.abs(S - Sw).max() <= 1e-5 * np.abs(Sw).max()
    # planted: v-head h reading k-head h // (n_v / n_k) differs
    qp, kp = np.repeat(q[0], 3, axis=0), np.repeat(k[0], 3, axis=0)
    bad, _ = O.ssm_delta_step(qp, kp, v[0], al[0], bt[0], a_log, dt, st, 0.3)
    assert np.abs(bad - want).max() > 1e-2
    # no decay (a_log = 0) and beta = +40 (sigmoid = 1): kn^T S' == v
    z = np.zeros_like(a_log)
    _, S1 = O.ssm_delta_step(q[0], k[0], v[0], al[0], np.full(6, 40.0, np.float32), z, dt,
                             st, 0.3)
    for h in range(6):
        kn = k[0][h % 2].astype(np.float64)
        kn /= np.linalg.norm(kn)
        assert np.abs(kn @ S1[h] - v[0][h]).max() <= 1e-5 * max(1.0, np.abs(v[0][h]).max())
    # beta = -80 (sigmoid underflows to 0): only the decay is applied
    _, S2 = O.ssm_delta_step(q[0], k[0], v[0], al[0], np.full(6, -80.0, np.float32), a_log,
                             dt, st, 0.3)
    for h in range(6):
        x = float(al[0][h]) + float(dt[h])
        g = min(float(a_log[h]) * (np.log1p(np.exp(-abs(x))) + max(x, 0.0)), 0.0)
        assert np.abs(S2[h] - st[h] * np.exp(g)).max() <= 1e-6
    # conv: two chunks == one pass; tap 0 pairs with the oldest input
    x = rng.standard_normal((9, 5)).astype(np.float32)
    w = rng.standard_normal((5, 4)).astype(np.float32)
    one, t1, l1 = O.ssm_conv(x, w, None, 0)
    a, ta, la = O.ssm_conv(x[:4], w, None, 0)
    b, tb, lb = O.ssm_conv(x[4:], w, ta, la)
    assert bits_equal(np.concatenate([a, b]), one) and l1 == lb == 3 and bits_equal(t1, tb)
    f64 = np.zeros((9, 5))
    for t in range(9):
        for j in range(4):
            if t - 3 + j >= 0:
                f64[t] += x[t - 3 + j].astype(np.float64) * w[:, j]
    assert np.abs(one - f64).max() <= 1e-5 * np.abs(f64).max()
    rev, _, _ = O.ssm_conv(x, w[:, ::-1].copy(), None, 0)
    assert np.abs(rev - f64).max() > 1e-2


def test_golden_ssm():
    """The reference's own scan and conv outputs (tests/golden/ref_vectors.npz)."""
    g = golden("ref_vectors.npz")
    out, st = O.ssm_scan(g["ssm_q"], g["ssm_k"], g["ssm_v"], g["ssm_alpha"], g["ssm_beta"],
                         g["ssm_a_log"], g["ssm_dt_bias"], g["ssm_state"], 0.125)
    assert bits_equal(out, g["ssm_out"]) and bits_equal(st, g["ssm_state_out"])
    o1, t1, l1 = O.ssm_conv(g["conv_x"][:2], g["conv_w"], None, 0)
    o2, t2, _ = O.ssm_conv(g["conv_x"][2:], g["conv_w"], t1, l1)
    assert bits_equal(np.concatenate([o1, o2]), g["conv_out"]) and bits_equal(t2, g["conv_tail"])


def _ssm_layer_case(rng, dts, n_embd, n_k, n_v, d, K):
    from aero_amd import workloads as W
    inner, qkv = n_v * d, 2 * n_k * d + n_v * d
    shapes = [(qkv, n_embd), (inner, n_embd), (n_v, n_embd), (n_v, n_embd), (n_embd, inner)]
    ws = [(rng.standard_normal((r, c)) / np.sqrt(c)).astype(np.float32) if t == 0
          else W.weight_table(t, r, c, rng) for t, (r, c) in zip(dts, shapes)]
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return dict(dts=list(dts), weights=ws, a_log=(-np.abs(f(n_v)) * 0.5).astype(np.float32),
                dt_bias=f(n_v), conv1d=(f(qkv, K) * 0.5).astype(np.float32),
                norm=(1 + f(d) * 0.1).astype(np.float32), n_k=n_k, d=d, inner=inner,
                eps=1e-6, norm_eps=1e-6)


@pytest.mark.parametrize("dts,n_embd,n_k,n_v,d,K", [
    ((0, 0, 0, 0, 0), 48, 2, 4, 16, 4),            # every projection fp32 (aero_ssm_forward)
    ((8, 8, 8, 8, 8), 64, 1, 2, 32, 4),            # Q8_0
    ((12, 12, 8, 8, 12), 256, 2, 4, 64, 3),        # Q4_K with Q8_0 gates, kernel 3
    ((14, 0, 0, 0, 14), 256, 1, 2, 128, 4),        # Q6_K with fp32 gate / alpha / beta
])
def test_ssm_forward_matches_compiled_reference(dts, n_embd, n_k, n_v, d, K):
    """The oracle's composition of one gated-DeltaNet layer (cpuref.ssm_forward)
    against aero_ssm_forward_q compiled from src/ssm.cpp: two calls of 5 and
    3 tokens carrying the conv history and the state, <= 1e-5 of scale (the
    reference sums its fp32 projections and the gated norm in float32, its
    quantised dots with -ffast-math)."""
    if R.ssm() is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(n_embd + d + K)
    case = _ssm_layer_case(rng, dts, n_embd, n_k, n_v, d, K)
    qkv = 2 * n_k * d + n_v * d
    tail, tl = np.zeros((K - 1, qkv), np.float32), 0
    rtail, rtl = tail, 0
    st = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
    rst = st
    for T in (5, 3):
        x = rng.standard_normal((T, n_embd)).astype(np.float32)
        out, tail, tl, st = O.ssm_forward(x, tail=tail, tail_len=tl, state=st, **case)
        rout, rtail, rtl, rst = R.ssm_forward(x, tail=rtail, tail_len=rtl, state=rst, **case)
        assert tl == rtl == min(K - 1, 8 if T == 3 else 5)
        assert rel_to_scale(out, rout) <= 1e-5, (T, rel_to_scale(out, rout))
        assert rel_to_scale(st, rst) <= 1e-5
        # the history holds raw projections: equal to their summation order
        assert rel_to_scale(tail[:tl], rtail[:rtl]) <= 1e-5


# ------------------------------------------------- dense fp32 and argmax
DENSE_SHAPES = ((1, 1, 1), (1, 7, 5), (1, 64, 896), (3, 33, 130), (5, 17, 4096), (2, 9, 4099))


@ref_built
def test_dense_matvec_matmul_match_compiled_reference():
    """cr_dense_matvec / cr_dense_matmul equal the reference's aero_tensor_matvec
    / aero_tensor_matmul (src/tensor.cpp:65-92,209-231) bit for bit, for one
    and several tokens and ragged widths, whatever the reference's thread
    count."""
    rng = np.random.default_rng(31)
    for n_tok, n_rows, n_cols in DENSE_SHAPES:
        w = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
        X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
        want = R.dense_matmul(w, X, threads=1)
        assert bits_equal(O.dense_matmul(w, X), want), (n_tok, n_rows, n_cols)
        assert bits_equal(R.dense_matmul(w, X, threads=4), want)
        if n_tok == 1:
            assert bits_equal(O.dense_matvec(w, X[0]), want[0])


def test_dense_matmul_is_the_product():
    """The fp32 sums are the float64 product to 5e-6 of scale; a planted
    regrouping (one product at a time in the one-token matvec) differs in
    the last bits somewhere, so the bit-exact checks above would catch it."""
    rng = np.random.default_rng(32)
    for n_tok, n_rows, n_cols in DENSE_SHAPES:
        w = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
        X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
        exact = X.astype(np.float64) @ w.astype(np.float64).T
        assert rel_to_scale(O.dense_matmul(w, X), exact) <= 5e-6
    w = rng.standard_normal((256, 4096)).astype(np.float32)
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    serial = np.empty(256, np.float32)
    for r in range(256):
        acc = np.float32(0)
        for p in (w[r] * x[0]):
            acc = np.float32(acc + p)
        serial[r] = acc
    assert not bits_equal(serial, O.dense_matvec(w, x[0]))


ARGMAX_CASES = [
    [3.0, 1.0, 3.0, 2.0],                         # first of equal maxima
    [float("nan"), 5.0, 7.0],                      # NaN at 0: index 0
    [1.0, float("nan"), 0.5, float("nan"), 2.0],   # NaN elsewhere never taken
    [-0.0, 0.0, -0.0],                             # signed zeros are equal
    [-np.inf, -np.inf, -np.inf],
    [-np.inf, np.inf, np.inf],
    [2.5],
]


@ref_built
def test_argmax_matches_compiled_reference():
    rng = np.random.default_rng(33)
    cases = [np.array(c, np.float32) for c in ARGMAX_CASES]
    cases += [rng.standard_normal(n).astype(np.float32) for n in (2, 1000, 151936)]
    t = rng.integers(0, 8, 5000).astype(np.float32)          # many ties
    cases.append(t)
    for v in cases:
        assert O.argmax(v) == R.argmax(v), v[:8]


def test_argmax_closed_forms():
    """First index of the largest value (np.argmax) on NaN-free input; 0 when
    v[0] is NaN; NaN elsewhere skipped."""
    rng = np.random.default_rng(34)
    for n in (1, 2, 77, 5000):
        v = rng.integers(-3, 4, n).astype(np.float32)
        assert O.argmax(v) == int(np.argmax(v))
    assert O.argmax(np.array(ARGMAX_CASES[1], np.float32)) == 0
    assert O.argmax(np.array(ARGMAX_CASES[2], np.float32)) == 4
    assert O.argmax(np.array(ARGMAX_CASES[3], np.float32)) == 0


def test_sigmoid_gate_closed_form_and_silu_relation():
    """The attention output gate 1/(1+exp(-g)) (src/attention_layer.cpp:
    262-263): float64 closed form, and v * sigmoid(v) equals the oracle's silu
    (itself the compiled reference's bit for bit) exactly."""
    rng = np.random.default_rng(35)
    v = (rng.standard_normal(5000) * 8).astype(np.float32)
    s = O.act(O.ACT_SIGMOID, v)
    exact = 1.0 / (1.0 + np.exp(-v.astype(np.float64)))
    assert np.abs(s - exact).max() <= 2e-7
    assert bits_equal((v * s).astype(np.float32), O.act(O.ACT_SILU, v))
    # the gate multiplies the attention output: sigmoid(g) * a, in either order
    a = rng.standard_normal(5000).astype(np.float32)
    assert bits_equal(O.act_mul(O.ACT_SIGMOID, v, a), (a * s).astype(np.float32))
