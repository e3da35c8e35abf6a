"""GPU: the reference-shaped modules (aero_amd.transformer_native,
aero_amd.tensor_native, aero_amd.native) behave like engine/transformer_native.py,
engine/tensor_native.py and engine/native.py, following the reference's own
suites tests/test_transformer_native.py, tests/test_tensor_native.py and
tests/test_quant_native_extra.py, with the oracle standing where those suites
use the numpy module.
"""
import math
import os
import struct

import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import native as NK
from aero_amd import tensor_native as TN
from aero_amd import transformer_native as N

pytestmark = pytest.mark.gpu


# ---------------------------------------------- tests/test_transformer_native.py
def test_transformer_native_rope_tables(hip, oracle):
    rng = np.random.default_rng(20261015)
    for label, nd, ff in (("full", None, None), ("partial-32", 32, None),
                          ("full + freq_factors", None, np.concatenate(
                              [np.ones(32, np.float32), np.full(32, 1e30, np.float32)]))):
        positions = rng.integers(0, 500, size=7).astype(np.int32)
        wc, ws = oracle.rope_tables(64, positions, 10000.0, nd, ff)
        gc, gs = N.rope_tables(64, positions, 10000.0, nd, freq_factors=ff)
        assert gc.shape == wc.shape, label
        assert max(rel_to_scale(gc, wc), rel_to_scale(gs, ws)) < RTOL, label
    with pytest.raises(ValueError):
        N.rope_tables(64, np.arange(3), 1e4, None, freq_factors=np.ones(5, np.float32))


def test_transformer_native_apply_rope(hip, oracle):
    rng = np.random.default_rng(20261015)
    Tn, H, D = 5, 3, 16
    x = rng.standard_normal((Tn, H, D)).astype(np.float32)
    positions = np.repeat(np.arange(Tn), H).astype(np.int32)
    ctab, stab = oracle.rope_tables(D, np.arange(Tn), 10000.0)
    for mode in (N.ROPE_NEOX, N.ROPE_INTERLEAVED):
        want = oracle.apply_rope(x, ctab, stab, positions, mode)
        got = N.apply_rope(x, ctab, stab, positions=positions, mode=mode)
        assert got.shape == x.shape
        assert bits_equal(got, want)  # same table: bit-exact
    c8, s8 = oracle.rope_tables(D, np.arange(Tn), 10000.0, 8)
    got = N.apply_rope(x, c8, s8, positions=positions, mode=N.ROPE_NEOX)
    assert bits_equal(got, oracle.apply_rope(x, c8, s8, positions, 0))
    assert bits_equal(got[..., 8:], x[..., 8:])
    # a copy, not in place
    assert not bits_equal(got, x)
    with pytest.raises(ValueError):
        N.apply_rope(x, ctab, stab, positions=positions + 10)


def test_transformer_native_norms_and_acts(hip, oracle):
    rng = np.random.default_rng(20261015)
    D = 16
    Xn = (rng.standard_normal((6, D)) * 2.0).astype(np.float32)
    wt = (rng.standard_normal(D) + 2.0).astype(np.float32)
    assert rel_to_scale(N.rmsnorm_rows(Xn, wt, 1e-6), oracle.rmsnorm_rows(Xn, wt, 1e-6)) < RTOL
    assert rel_to_scale(N.l2norm_rows(Xn, wt, 1e-6), oracle.l2norm_rows(Xn, wt, 1e-6)) < RTOL
    # 3-D input: every (token, head) row is normalised
    X3 = rng.standard_normal((4, 3, D)).astype(np.float32)
    assert rel_to_scale(N.rmsnorm_rows(X3, wt, 1e-6), oracle.rmsnorm_rows(X3, wt, 1e-6)) < RTOL
    z = (rng.standard_normal(401) * 5.0).astype(np.float32)
    up = rng.standard_normal(401).astype(np.float32)
    assert rel_to_scale(N.gelu(z), oracle.act(1, z)) < RTOL
    assert rel_to_scale(N.silu(z), oracle.act(0, z)) < RTOL
    assert rel_to_scale(N.swiglu(z, up), oracle.act_mul(0, z, up)) < RTOL
    zc = z.copy()
    N.gelu(zc)
    assert bits_equal(zc, z)  # returns a copy


# ---------------------------------------------- tests/test_tensor_native.py
def test_tensor_native_elementwise(hip, oracle):
    rng = np.random.default_rng(7)
    n = 2560
    xs = rng.standard_normal(n).astype(np.float32)
    up = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) + 1.5).astype(np.float32)
    for name, kind in (("gelu", 1), ("silu", 0)):
        b = getattr(TN, name)(xs.copy())
        assert np.abs(b - oracle.act(kind, xs)).max() < 1e-5, name
    b = TN.swiglu(xs.copy(), up.copy())
    assert np.abs(b - oracle.act_mul(0, xs, up)).max() < 1e-5
    assert np.allclose(TN.mul(xs.copy(), g.copy()), xs * g, atol=1e-6)
    # in place on a contiguous float32 input (engine/tensor_native.py:153-160)
    buf = xs.copy()
    ret = TN.silu(buf)
    assert ret.ctypes.data == buf.ctypes.data
    assert not bits_equal(buf, xs)


def test_tensor_native_closed_forms(hip):
    for xv in (0.0, 1.0, 3.0, -2.5):
        got = float(TN.gelu(np.array([xv], np.float32))[0])
        want = 0.5 * xv * (1.0 + math.erf(xv / math.sqrt(2.0)))
        tanh = 0.5 * xv * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (xv + 0.044715 * xv ** 3)))
        assert abs(got - want) < 1e-6 and (xv == 0.0 or abs(got - tanh) > 1e-7)
    for xv in (0.0, 1.0, -1.0, 5.0):
        got = float(TN.silu(np.array([xv], np.float32))[0])
        assert abs(got - xv / (1.0 + math.exp(-xv))) < 1e-6


def test_tensor_native_norms(hip):
    rng = np.random.default_rng(7)
    xs = rng.standard_normal(2560).astype(np.float32)
    g = (rng.standard_normal(2560) + 1.5).astype(np.float32)
    out = TN.rmsnorm(xs.copy(), g.copy(), 1e-6)
    want = xs / np.sqrt((xs.astype(np.float64) ** 2).mean() + 1e-6) * g
    assert rel_to_scale(out, want) < 1e-6
    v = rng.standard_normal(64).astype(np.float32)
    assert abs(float(np.linalg.norm(TN.l2norm(v, None, eps=1e-6))) - 1.0) < 1e-5
    v_sub = np.full(64, 1e-9, np.float32)
    got_norm = float(np.linalg.norm(TN.l2norm(v_sub.copy(), None, eps=1e-6).astype(np.float64)))
    want_norm = float(np.linalg.norm(v_sub.astype(np.float64))) / 1e-6
    assert abs(got_norm - want_norm) / want_norm < 1e-3
    t = rng.standard_normal((3, 32)).astype(np.float32)
    r = TN.rmsnorm_rows(t, 1e-6)
    assert r is t or r.ctypes.data == t.ctypes.data
    assert np.allclose(np.sqrt((t.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-3)


def test_tensor_native_refusals(hip):
    for fn, args in ((TN.mul, (np.zeros(4, np.float32), np.zeros(5, np.float32))),
                     (TN.rmsnorm, (np.zeros(4, np.float32), np.zeros(5, np.float32), 1e-6)),
                     (TN.swiglu, (np.zeros(4, np.float32), np.zeros(3, np.float32)))):
        with pytest.raises((ValueError, TypeError)):
            fn(*args)
    with pytest.raises(ValueError):
        TN.silu(np.zeros(0, np.float32))
    with pytest.raises(ValueError):
        TN.rmsnorm_rows(np.zeros(4, np.float32), 1e-6)
    r64 = TN.silu(np.arange(8, dtype=np.float64))
    assert r64.dtype == np.float32


def test_tensor_native_dense_and_argmax(hip, oracle):
    """matvec / matmul / argmax (src/tensor.cpp:65-92,180-186): bit-identical to
    the oracle's restatement of the reference's sums, and to the reference's
    own compiled functions where oracle/_ref is built."""
    from oracle import refbind
    rng = np.random.default_rng(41)
    for n_tok, n_rows, n_cols in ((1, 1, 1), (1, 7, 5), (1, 896, 896), (1, 300, 4099),
                                  (3, 33, 130), (5, 257, 4096), (2, 9, 1027)):
        w = rng.standard_normal((n_rows, n_cols)).astype(np.float32)
        X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
        print(f"tensor_native dense tokens={n_tok} rows={n_rows} cols={n_cols}", flush=True)
        want = oracle.dense_matmul(w, X)
        got = TN.matvec(w, X[0]) if n_tok == 1 else TN.matmul(w, X, threads=3)
        assert bits_equal(got.reshape(want.shape), want)
        if n_tok == 1:
            assert bits_equal(TN.matmul(w, X), want)
        if refbind.available():
            assert bits_equal(want, refbind.dense_matmul(w, X))
    nan, inf = float("nan"), float("inf")
    cases = [np.array(c, np.float32) for c in
             ([3, 1, 3, 2], [nan, 5, 7], [1, nan, 0.5, nan, 2], [-0.0, 0.0, -0.0],
              [-inf, -inf], [-inf, inf, inf], [2.5])]
    cases += [rng.standard_normal(n).astype(np.float32) for n in (2, 1025, 151936)]
    cases.append(rng.integers(0, 8, 100000).astype(np.float32))
    for v in cases:
        assert TN.argmax(v) == oracle.argmax(v), v[:6]
        if refbind.available():
            assert oracle.argmax(v) == refbind.argmax(v)
    assert TN.threads() == min(os.cpu_count() or 1, 8)
    with pytest.raises(ValueError):
        TN.matvec(np.zeros((3, 4), np.float32), np.zeros(5, np.float32))
    with pytest.raises(ValueError):
        TN.argmax(np.zeros(0, np.float32))


def test_reference_loader_binds_the_library(hip):
    """The reference's loader (engine/tensor_native.py:41-71) sets these
    argtypes on every symbol and treats a missing one as an unusable library;
    bound the same way, libaero_hip.so has every symbol and they compute."""
    import ctypes
    from ctypes import POINTER, c_float, c_int, c_int64

    from aero_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    cp = POINTER(c_float)
    lib.aero_tensor_matvec.argtypes = [cp, cp, cp, c_int64, c_int64, c_int]
    lib.aero_tensor_matvec.restype = c_int
    lib.aero_tensor_matmul.argtypes = [cp, cp, cp, c_int64, c_int64, c_int64, c_int]
    lib.aero_tensor_matmul.restype = c_int
    for name in ("silu", "gelu", "softmax"):
        f = getattr(lib, "aero_tensor_" + name)
        f.argtypes = [cp, c_int64]
        f.restype = c_int
    lib.aero_tensor_mul.argtypes = [cp, cp, c_int64]
    lib.aero_tensor_mul.restype = c_int
    lib.aero_tensor_swiglu.argtypes = [cp, cp, c_int64]
    lib.aero_tensor_swiglu.restype = c_int
    lib.aero_tensor_rmsnorm.argtypes = [cp, cp, cp, c_int64, c_float]
    lib.aero_tensor_rmsnorm.restype = c_int
    lib.aero_tensor_l2norm.argtypes = [cp, cp, cp, c_int64, c_float, c_int]
    lib.aero_tensor_l2norm.restype = c_int
    lib.aero_tensor_rmsnorm_rows.argtypes = [cp, c_int64, c_int64, c_float]
    lib.aero_tensor_rmsnorm_rows.restype = c_int
    lib.aero_tensor_argmax.argtypes = [cp, c_int64]
    lib.aero_tensor_argmax.restype = c_int
    lib.aero_tensor_threads.argtypes = []
    lib.aero_tensor_threads.restype = c_int
    w = np.arange(12, dtype=np.float32).reshape(3, 4)
    x = np.ones(4, np.float32)
    y = np.empty(3, np.float32)
    p = lambda a: a.ctypes.data_as(cp)  # noqa: E731
    assert lib.aero_tensor_matvec(p(w), p(x), p(y), 3, 4, 0) == 1
    assert y.tolist() == [6.0, 22.0, 38.0]
    assert lib.aero_tensor_argmax(p(y), 3) == 2
    assert lib.aero_tensor_argmax(p(y), 0) == -1
    assert lib.aero_tensor_matvec(p(w), p(x), p(y), 0, 4, 0) == 0
    assert lib.aero_tensor_threads() >= 1


# ---------------------------------------------- tests/test_quant_native_extra.py
def f16(v: float) -> bytes:
    return struct.pack("<e", v)


@pytest.mark.parametrize("type_id,bb,bv", [(8, 34, 32), (12, 144, 256), (13, 176, 256),
                                            (14, 210, 256), (23, 136, 256)])
def test_native_dequant(hip, oracle, type_id, bb, bv):
    rng = np.random.default_rng(4)
    assert type_id in NK.NATIVE_TYPES
    assert NK.block_bytes(type_id) == bb and NK.block_values(type_id) == bv
    NB = 4
    buf = bytearray(rng.integers(0, 256, size=NB * bb, dtype=np.uint8).tobytes())
    for b in range(NB):
        off = b * bb
        if type_id == 14:
            buf[off + 208:off + 210] = f16(0.02 * (b + 1))
        else:
            buf[off:off + 2] = f16(0.02 * (b + 1))
            if type_id in (12, 13):
                buf[off + 2:off + 4] = f16(0.01 * (b + 1))
    raw = bytes(buf)
    want = oracle.dequant(type_id, np.frombuffer(raw, np.uint8), NB * bv)
    for r in (raw, bytearray(raw), memoryview(bytearray(raw)), np.frombuffer(raw, np.uint8)):
        got = NK.dequant(type_id, r, (NB, bv))
        assert got.shape == (NB, bv)
        assert bits_equal(got.reshape(-1), want)
        assert np.isfinite(got).all()
    with pytest.raises(ValueError):
        NK.dequant(type_id, raw[:bb], (NB * bv,))


def test_native_dequant_refuses_other_types(hip):
    with pytest.raises(ValueError):
        NK.dequant(2, bytes(18), (32,))          # Q4_0: not a native type
    with pytest.raises(TypeError):
        NK.dequant(NK.DTYPE_Q8_0, [1, 2, 3], (32,))
