"""GPU: the reference-shaped modules (aero_amd.transformer_native,
aero_amd.tensor_native, aero_amd.native) behave like engine/transformer_native.py,
engine/tensor_native.py and engine/native.py, following the reference's own
suites tests/test_transformer_native.py, tests/test_tensor_native.py and
tests/test_quant_native_extra.py, with the oracle standing where those suites
use the numpy module.
"""
import math
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
