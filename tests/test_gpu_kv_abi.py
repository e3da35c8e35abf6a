"""GPU: the KV cache host ABI of src/kv.cpp (aero_kv_write_vec / read_vec /
ring_indices / ring_rotate / span_error / slot_*), bound with the reference
suite's own argtypes (tests/test_kv_native.py:54-64) and checked as that
suite checks it: byte-exact int8 and int4 codes (low nibble first) and
scales, bit-exact reads, the span error metric, the ring's chronological
order, the refusals. The oracle (cpuref's kv_write_vec / kv_read_vec,
restating src/kv.cpp) and, where oracle/_ref is built, the reference's own
compiled functions are the expected values. Slots live in HBM here; they
are checked against the reference's KvSlot round trip and, through
aero_hip_kv_slot_view, against the attention entry point reading them.
"""
import ctypes
from ctypes import POINTER, c_float, c_int, c_int64, c_void_p

import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import _lib
from oracle import refbind as R

pytestmark = pytest.mark.gpu

fp = POINTER(c_float)


@pytest.fixture(scope="module")
def lib(hip):
    L = ctypes.CDLL(_lib.LIB_PATH)
    L.aero_kv_write_vec.argtypes = [c_int, fp, c_int64, c_void_p, fp]
    L.aero_kv_write_vec.restype = c_int
    L.aero_kv_read_vec.argtypes = [c_int, c_void_p, fp, c_int64, fp]
    L.aero_kv_read_vec.restype = c_int
    L.aero_kv_ring_rotate.argtypes = [c_int64, c_int64, c_int64, POINTER(c_int64)]
    L.aero_kv_ring_rotate.restype = c_int
    L.aero_kv_ring_indices.argtypes = [c_int64, c_int64, POINTER(c_int64)]
    L.aero_kv_ring_indices.restype = c_int
    L.aero_kv_span_error.argtypes = [c_int, c_void_p, fp, c_int64, fp, fp]
    L.aero_kv_span_error.restype = c_int
    return L


def nbytes(dt, dim):
    return dim * 4 if dt == 0 else (dim // 2 if dt == 2 else dim)


def write(lib, dt, x):
    q = np.zeros(nbytes(dt, x.size), np.uint8)
    s = np.zeros(1, np.float32)
    ok = lib.aero_kv_write_vec(dt, x.ctypes.data_as(fp), x.size, q.ctypes.data,
                               s.ctypes.data_as(fp))
    return ok, q, float(s[0])


def read(lib, dt, q, s, dim):
    out = np.zeros(dim, np.float32)
    sc = np.array([s], np.float32)
    ok = lib.aero_kv_read_vec(dt, q.ctypes.data, sc.ctypes.data_as(fp), dim,
                              out.ctypes.data_as(fp))
    return ok, out


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("dim", [2, 64, 128, 130, 256])
def test_write_read_byte_exact(lib, oracle, dt, dim):
    rng = np.random.default_rng(11 + dim)
    for scale in (2.5, 1e-3, 0.0):
        x = (rng.standard_normal(dim) * scale).astype(np.float32)
        print(f"kv vec dt={dt} dim={dim} scale={scale}", flush=True)
        ok, q, s = write(lib, dt, x)
        assert ok == 1
        wq, ws = oracle.kv_write_vec(dt, x)
        assert np.array_equal(q, wq) and (dt == 0 or np.float32(s) == np.float32(ws))
        okr, back = read(lib, dt, q, s, dim)
        assert okr == 1 and bits_equal(back, oracle.kv_read_vec(dt, q, s, dim))
        if R.available():
            rq, rs = R.kv_write_vec(dt, x)
            assert np.array_equal(q, rq) and (dt == 0 or np.float32(s) == np.float32(rs))
            assert bits_equal(back, R.kv_read_vec(dt, q, s, dim))
        if dt == 0:
            assert bits_equal(back, x)


def test_int4_low_nibble_first_and_sign_extension(lib):
    """src/kv.cpp:30-46 / include/aero/kv.hpp:80-110: codes -7..7 as (v & 15),
    low nibble first; read back sign-extended from 4 bits."""
    x = np.array([7, -7, 1, -1, 0, 3, -3, 7], np.float32)
    ok, q, s = write(lib, 2, x)
    assert ok == 1 and s == 1.0
    assert q.tolist() == [0x97, 0xF1, 0x30, 0x7D]
    okr, back = read(lib, 2, q, s, 8)
    assert okr == 1 and back.tolist() == x.tolist()


def test_span_error_metric(lib):
    """max|x - read(q)| / max|x| (1e-9 for all-zero x), bit-exact with the
    reference; int4 is coarser than int8 (tests/test_kv_native.py:139-156)."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(128) * 2.5).astype(np.float32)
    errs = {}
    for dt in (0, 1, 2):
        ok, q, s = write(lib, dt, x)
        sc = np.array([s], np.float32)
        e = np.zeros(1, np.float32)
        assert lib.aero_kv_span_error(dt, q.ctypes.data, sc.ctypes.data_as(fp), x.size,
                                      x.ctypes.data_as(fp), e.ctypes.data_as(fp)) == 1
        back = read(lib, dt, q, s, x.size)[1]
        want = np.float32(np.abs(back - x).max()) / np.float32(np.abs(x).max())
        assert np.float32(e[0]) == np.float32(want)
        if R.available():
            assert np.float32(e[0]) == np.float32(R.kv_span_error(dt, q, s, x))
        errs[dt] = float(e[0])
    assert errs[0] == 0.0 and errs[2] > errs[1] > 0.0
    z = np.zeros(16, np.float32)
    ok, q, s = write(lib, 1, z)
    e = np.zeros(1, np.float32)
    sc = np.array([s], np.float32)
    assert lib.aero_kv_span_error(1, q.ctypes.data, sc.ctypes.data_as(fp), 16,
                                  z.ctypes.data_as(fp), e.ctypes.data_as(fp)) == 1
    assert e[0] == 0.0


def test_ring_rotation_and_indices(lib):
    """Index 0 is the oldest retained position (tests/test_kv_native.py:158-
    176): (start + i) % cap; the unwrapped ring is 0 .. n-1."""
    for cap, start in ((8, 3), (16, 7), (64, 0), (5, 4)):
        out = (c_int64 * cap)()
        assert lib.aero_kv_ring_rotate(cap, start, cap, out) == 1
        want = np.concatenate([np.arange(start, cap), np.arange(0, start)])
        assert np.array_equal(np.array(out[:]), want)
        if R.available():
            assert np.array_equal(R.kv_ring_rotate(cap, start, cap)[1], want)
    out = (c_int64 * 6)()
    assert lib.aero_kv_ring_indices(8, 6, out) == 1 and list(out) == list(range(6))
    assert lib.aero_kv_ring_rotate(8, 9, 8, (c_int64 * 8)()) == 0      # start >= cap
    assert lib.aero_kv_ring_rotate(8, 0, 9, (c_int64 * 9)()) == 0      # n > cap
    assert lib.aero_kv_ring_indices(4, 5, (c_int64 * 5)()) == 0


def test_refusals(lib):
    """Unknown dt, odd int4 dim, NULL buffers (tests/test_kv_native.py:178-
    189)."""
    x = np.ones(8, np.float32)
    assert lib.aero_kv_write_vec(7, x.ctypes.data_as(fp), 8, None, fp(c_float())) == 0
    xo = np.ones(7, np.float32)
    assert lib.aero_kv_write_vec(2, xo.ctypes.data_as(fp), 7, None, fp(c_float())) == 0
    assert lib.aero_kv_read_vec(2, np.zeros(4, np.uint8).ctypes.data, fp(c_float(1.0)), 7,
                                np.zeros(7, np.float32).ctypes.data_as(fp)) == 0
    assert lib.aero_kv_span_error(1, None, fp(c_float(1.0)), 8, x.ctypes.data_as(fp),
                                  fp(c_float())) == 0


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_slot_roundtrip_matches_reference_slot(hip, oracle, dt):
    """aero_kv_slot_new / write / read / bytes: every (phys, head) vector of
    an HBM slot reads back as the reference's KvSlot gives it (zeros where
    nothing was written), and bytes() is the reference's formula."""
    L = _lib.lib()
    cap, heads, dim = 6, 3, 64
    rng = np.random.default_rng(13 + dt)
    writes = [(p, h, (rng.standard_normal(dim) * 3).astype(np.float32))
              for p, h in ((0, 0), (0, 2), (3, 1), (5, 2), (3, 1))]   # (3, 1) rewritten
    sl = L.aero_kv_slot_new(cap, heads, dim, dt, 0)
    assert sl
    try:
        for p, h, x in writes:
            assert L.aero_kv_slot_write(sl, p, h, x.ctypes.data_as(fp)) == 1
        got = np.zeros((cap, heads, dim), np.float32)
        for p in range(cap):
            for h in range(heads):
                assert L.aero_kv_slot_read(sl, p, h, got[p, h].ctypes.data_as(fp)) == 1
        want = np.zeros((cap, heads, dim), np.float32)
        for p, h, x in writes:
            q, s = oracle.kv_write_vec(dt, x)
            want[p, h] = oracle.kv_read_vec(dt, q, s, dim)
        assert bits_equal(got, want)
        vb = {0: dim * 4, 1: dim, 2: dim // 2}[dt]
        assert L.aero_kv_slot_bytes(sl) == cap * heads * vb + (cap * heads * 4 if dt else 0)
        if R.available():
            rb, rwant = R.kv_slot_roundtrip(cap, heads, dim, dt, writes)
            assert bits_equal(got, rwant) and rb == L.aero_kv_slot_bytes(sl)
        # out of range phys or head, and NULL: refused
        x0 = writes[0][2]
        assert L.aero_kv_slot_write(sl, cap, 0, x0.ctypes.data_as(fp)) == 0
        assert L.aero_kv_slot_write(sl, 0, heads, x0.ctypes.data_as(fp)) == 0
        assert L.aero_kv_slot_read(sl, -1, 0, got[0, 0].ctypes.data_as(fp)) == 0
    finally:
        L.aero_kv_slot_free(sl)
    assert L.aero_kv_slot_bytes(None) == -1
    assert not L.aero_kv_slot_new(4, 2, 7, 2, 0)       # int4 needs an even dim
    assert not L.aero_kv_slot_new(0, 2, 8, 1, 0)


def test_slot_view_feeds_attention(hip, oracle):
    """Two int8 slots (K and V) filled through the host ABI are read in HBM by
    aero_hip_attention through aero_hip_kv_slot_view: the result equals the
    oracle's attention over the slots' dequantised vectors."""
    from aero_amd.device import DeviceArray as DA
    L = _lib.lib()
    S, HK, H, D = 40, 2, 4, 64
    rng = np.random.default_rng(14)
    K = rng.standard_normal((S, HK, D)).astype(np.float32)
    V = rng.standard_normal((S, HK, D)).astype(np.float32)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    slots = [L.aero_kv_slot_new(S, HK, D, 1, 0) for _ in range(2)]
    try:
        deq = []
        for sl, X in zip(slots, (K, V)):
            for p in range(S):
                for h in range(HK):
                    xv = np.ascontiguousarray(X[p, h])
                    assert L.aero_kv_slot_write(sl, p, h, xv.ctypes.data_as(fp)) == 1
            back = np.zeros((S, HK, D), np.float32)
            for p in range(S):
                for h in range(HK):
                    q8, s8 = oracle.kv_write_vec(1, X[p, h])
                    back[p, h] = oracle.kv_read_vec(1, q8, s8, D)
            deq.append(back)
        views = []
        for sl in slots:
            qp, sp = c_void_p(), fp()
            cap, heads, dim = c_int64(), c_int64(), c_int64()
            dt, ring = c_int(), c_int()
            assert L.aero_hip_kv_slot_view(sl, ctypes.byref(qp), ctypes.byref(sp),
                                           ctypes.byref(cap), ctypes.byref(heads),
                                           ctypes.byref(dim), ctypes.byref(dt),
                                           ctypes.byref(ring)) == 1
            assert (cap.value, heads.value, dim.value, dt.value, ring.value) == (S, HK, D, 1, 0)
            views.append((qp.value, ctypes.cast(sp, c_void_p).value))
        dq = DA.from_numpy(q)
        out = DA.empty((1, H, D))
        ws_b = L.aero_hip_attention_workspace(1, H, HK, D, D, S)
        ws = DA.empty((max(ws_b, 16),), np.uint8)
        pos = DA.from_numpy(np.array([S - 1], np.int32))
        assert L.aero_hip_attention(dq.ptr, 1, views[0][0], views[0][1], views[1][0],
                                    views[1][1], out.ptr, 1, H, HK, D, D,
                                    float(1.0 / np.sqrt(D)), pos.ptr, None, S, 0, ws.ptr,
                                    ws_b, None) == 1, _lib.last_error()
        want = oracle.attention_tiled(q, deq[0], deq[1], 1.0 / np.sqrt(D),
                                      qpos=np.array([S - 1], np.int32))
        assert rel_to_scale(out.numpy(), want) <= RTOL
    finally:
        for sl in slots:
            L.aero_kv_slot_free(sl)
