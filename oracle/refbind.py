"""ctypes binding of the reference's own hot-path C++ built into oracle/_ref/.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). `make -C oracle ref`
compiles src/kernels.cpp and src/transformer.cpp + src/tensor.cpp of the
reference tree into oracle/_ref/; those libraries export the reference's C ABI
(src/kernels.cpp:560-603, src/tensor.cpp:205-304, src/transformer.cpp:
223-284). This module loads them when present and returns None otherwise, so
callers skip the cross-check rather than fail.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint8

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")
KERNELS = os.path.join(REF_DIR, "libref_kernels.so")
TRANSFORMER = os.path.join(REF_DIR, "libref_transformer.so")
KV = os.path.join(REF_DIR, "libref_kv.so")
GGUF = os.path.join(REF_DIR, "libref_gguf.so")
SSM = os.path.join(REF_DIR, "libref_ssm.so")

_k = None
_t = None
_v = None
_g = None
_s = None


def kernels():
    global _k
    if _k is None and os.path.exists(KERNELS):
        L = ctypes.CDLL(KERNELS)
        L.aero_dequant_ref.argtypes = [c_int, POINTER(c_uint8), c_int64,
                                       POINTER(c_float), c_int64]
        L.aero_dequant_ref.restype = c_int
        L.aero_dequant_threaded.argtypes = [c_int, POINTER(c_uint8), c_int64,
                                            POINTER(c_float), c_int64, c_int]
        L.aero_dequant_threaded.restype = c_int
        L.aero_matvec.argtypes = [c_int, POINTER(c_uint8), POINTER(c_float),
                                  POINTER(c_float), c_int64, c_int64, c_int]
        L.aero_matvec.restype = c_int
        L.aero_matmul.argtypes = [c_int, POINTER(c_uint8), POINTER(c_float),
                                  POINTER(c_float), c_int64, c_int64, c_int64, c_int]
        L.aero_matmul.restype = c_int
        _k = L
    return _k


def transformer():
    global _t
    if _t is None and os.path.exists(TRANSFORMER):
        L = ctypes.CDLL(TRANSFORMER)
        fp, ip = POINTER(c_float), POINTER(c_int32)
        L.aero_rope_tables.argtypes = [c_int64, ip, c_int64, c_float, c_int64, fp,
                                       c_int64, fp, fp]
        L.aero_rope_tables.restype = c_int64
        L.aero_apply_rope.argtypes = [fp, c_int64, c_int64, c_int64, fp, fp, ip, c_int]
        L.aero_apply_rope.restype = None
        L.aero_rmsnorm_rows.argtypes = [fp, fp, fp, c_int64, c_int64, c_float]
        L.aero_rmsnorm_rows.restype = None
        L.aero_l2norm_rows.argtypes = [fp, fp, fp, c_int64, c_int64, c_float]
        L.aero_l2norm_rows.restype = None
        for name in ("aero_gelu", "aero_silu"):
            getattr(L, name).argtypes = [fp, c_int64]
            getattr(L, name).restype = None
        L.aero_swiglu.argtypes = [fp, fp, c_int64]
        L.aero_swiglu.restype = None
        L.aero_tensor_mul.argtypes = [fp, fp, c_int64]
        L.aero_tensor_mul.restype = c_int
        L.aero_softmax_rows.argtypes = [fp, c_int64, c_int64]
        L.aero_softmax_rows.restype = None
        L.aero_tensor_matvec.argtypes = [fp, fp, fp, c_int64, c_int64, c_int]
        L.aero_tensor_matvec.restype = c_int
        L.aero_tensor_matmul.argtypes = [fp, fp, fp, c_int64, c_int64, c_int64, c_int]
        L.aero_tensor_matmul.restype = c_int
        L.aero_tensor_argmax.argtypes = [fp, c_int64]
        L.aero_tensor_argmax.restype = c_int
        L.aero_tensor_threads.argtypes = []
        L.aero_tensor_threads.restype = c_int
        L.aero_attention_tiled.argtypes = [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64,
                                           c_int64, c_float, ip, ip, c_int64, c_int, c_int64]
        L.aero_attention_tiled.restype = c_int
        L.aero_attention.argtypes = [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64,
                                     c_float, c_int64, c_int]
        L.aero_attention.restype = c_int
        _t = L
    return _t


def kv():
    global _v
    if _v is None and os.path.exists(KV):
        L = ctypes.CDLL(KV)
        fp = POINTER(c_float)
        L.aero_kv_write_vec.argtypes = [c_int, fp, c_int64, ctypes.c_void_p, fp]
        L.aero_kv_write_vec.restype = c_int
        L.aero_kv_read_vec.argtypes = [c_int, ctypes.c_void_p, fp, c_int64, fp]
        L.aero_kv_read_vec.restype = c_int
        i64p, vp = POINTER(c_int64), ctypes.c_void_p
        L.aero_kv_ring_indices.argtypes = [c_int64, c_int64, i64p]
        L.aero_kv_ring_indices.restype = c_int
        L.aero_kv_ring_rotate.argtypes = [c_int64, c_int64, c_int64, i64p]
        L.aero_kv_ring_rotate.restype = c_int
        L.aero_kv_span_error.argtypes = [c_int, vp, fp, c_int64, fp, fp]
        L.aero_kv_span_error.restype = c_int
        L.aero_kv_slot_new.argtypes = [c_int64, c_int64, c_int64, c_int, c_int]
        L.aero_kv_slot_new.restype = vp
        L.aero_kv_slot_free.argtypes = [vp]
        L.aero_kv_slot_free.restype = None
        L.aero_kv_slot_bytes.argtypes = [vp]
        L.aero_kv_slot_bytes.restype = c_int64
        L.aero_kv_slot_write.argtypes = [vp, c_int64, c_int64, fp]
        L.aero_kv_slot_write.restype = c_int
        L.aero_kv_slot_read.argtypes = [vp, c_int64, c_int64, fp]
        L.aero_kv_slot_read.restype = c_int
        _v = L
    return _v


def gguf():
    """The reference's GgufReader (src/gguf.cpp) through oracle/ref_gguf_shim.cpp."""
    global _g
    if _g is None and os.path.exists(GGUF):
        L = ctypes.CDLL(GGUF)
        vp, cp = ctypes.c_void_p, ctypes.c_char_p
        for name, res, args in (
                ("rg_open", vp, [cp, cp, c_int]), ("rg_close", None, [vp]),
                ("rg_arch", cp, [vp]), ("rg_file_size", c_int64, [vp]),
                ("rg_has", c_int, [vp, cp]), ("rg_get_int", c_int64, [vp, cp, c_int64]),
                ("rg_get_float", ctypes.c_double, [vp, cp, ctypes.c_double]),
                ("rg_get_str", c_int64, [vp, cp, cp, c_int64]),
                ("rg_int_array", c_int64, [vp, cp, POINTER(c_int64), c_int64]),
                ("rg_str_array_len", c_int64, [vp, cp]),
                ("rg_str_array_item", c_int64, [vp, cp, c_int64, cp, c_int64]),
                ("rg_n_tensors", c_int64, [vp]),
                ("rg_tensor", c_int, [vp, cp, POINTER(c_int), POINTER(c_int), POINTER(c_int64),
                                      POINTER(c_int64), POINTER(c_int64)]),
                ("rg_tensor_data", vp, [vp, cp])):
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _g = L
    return _g


def ssm():
    """The reference's gated-DeltaNet C ABI (src/ssm.cpp:151-210)."""
    global _s
    if _s is None and os.path.exists(SSM):
        L = ctypes.CDLL(SSM)
        fp = POINTER(c_float)
        L.aero_ssm_softplus.argtypes = [c_float]
        L.aero_ssm_softplus.restype = c_float
        L.aero_ssm_delta_step.argtypes = [fp] * 8 + [c_int, c_int, c_float, c_float, fp]
        L.aero_ssm_delta_step.restype = None
        L.aero_ssm_scan.argtypes = [fp] * 8 + [c_int] * 4 + [c_float, c_float, fp]
        L.aero_ssm_scan.restype = None
        L.aero_ssm_conv.argtypes = [fp, fp, fp, POINTER(c_int), fp, c_int, c_int, c_int]
        L.aero_ssm_conv.restype = None
        vp = ctypes.c_void_p
        L.aero_ssm_forward_q.argtypes = ([fp, POINTER(c_int), POINTER(vp), POINTER(c_int64)]
                                         + [fp] * 4 + [c_int] * 7 + [c_float, c_float, fp,
                                                                     POINTER(c_int), fp, fp,
                                                                     c_int])
        L.aero_ssm_forward_q.restype = c_int
        _s = L
    return _s


def ssm_delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """aero_ssm_delta_step: q, k already (n_heads, d). Returns (out, new state)."""
    f = lambda a: np.ascontiguousarray(a, np.float32)
    q, k, v = f(q), f(k), f(v)
    n, d = v.shape
    st = np.array(f(state), copy=True)
    out = np.zeros((n, d), np.float32)
    ssm().aero_ssm_delta_step(_f(q), _f(k), _f(v), _f(f(alpha)), _f(f(beta)), _f(f(a_log)),
                              _f(f(dt_bias)), _f(st), n, d, float(scale), float(eps), _f(out))
    return out, st


def ssm_scan(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    f = lambda a: np.ascontiguousarray(a, np.float32)
    q, k, v = f(q), f(k), f(v)
    T, n_k, d = q.shape
    n_v = v.shape[1]
    st = np.array(f(state), copy=True)
    outs = np.zeros((T, n_v, d), np.float32)
    ssm().aero_ssm_scan(_f(q), _f(k), _f(v), _f(f(alpha)), _f(f(beta)), _f(f(a_log)),
                        _f(f(dt_bias)), _f(st), T, n_k, n_v, d, float(scale), float(eps),
                        _f(outs))
    return outs, st


def ssm_forward(x, dts, weights, a_log, dt_bias, conv1d, norm, n_k: int, d: int, inner: int,
                eps: float, norm_eps: float, tail, tail_len: int, state, threads: int = 1):
    """aero_ssm_forward_q (src/ssm.cpp:262-352) on the same arguments as the
    oracle's cpuref.ssm_forward. Returns (out, tail, tail_len, state)."""
    f = lambda a: np.ascontiguousarray(a, np.float32)
    x = f(x)
    T, n_embd = x.shape
    n_v = inner // d
    qkv_w = 2 * n_k * d + inner
    K = conv1d.shape[1]
    keep = [f(w) if dt == 0 else np.ascontiguousarray(w, np.uint8).reshape(-1)
            for dt, w in zip(dts, weights)]
    wp = (ctypes.c_void_p * 5)(*[w.ctypes.data for w in keep])
    wl = (c_int64 * 5)(*[0 if dt == 0 else w.size for dt, w in zip(dts, keep)])
    dt = (c_int * 5)(*[int(t) for t in dts])
    tb = np.zeros((max(K - 1, 1), qkv_w), np.float32)
    if tail_len > 0:
        tb[:tail_len] = f(tail)[:tail_len]
    tl = c_int(int(tail_len))
    st = np.array(f(state), copy=True)
    out = np.zeros((T, n_embd), np.float32)
    rc = ssm().aero_ssm_forward_q(_f(x), dt, wp, wl, _f(f(a_log)), _f(f(dt_bias)), _f(f(conv1d)),
                                  _f(f(norm)), T, n_embd, inner, d, n_k, K, n_v, float(eps),
                                  float(norm_eps), _f(tb), ctypes.byref(tl), _f(st), _f(out),
                                  int(threads))
    if rc != 0:
        raise ValueError(f"aero_ssm_forward_q refused ({rc})")
    return out, tb[:max(K - 1, 0)], int(tl.value), st


def ssm_conv(x, w, tail, tail_len: int):
    f = lambda a: np.ascontiguousarray(a, np.float32)
    x, w = f(x), f(w)
    T, C = x.shape
    kernel = w.shape[1]
    tb = np.zeros((max(kernel - 1, 1), C), np.float32)
    if tail_len > 0:
        tb[:tail_len] = f(tail)[:tail_len]
    out = np.zeros((T, C), np.float32)
    tl = c_int(int(tail_len))
    ssm().aero_ssm_conv(_f(x), _f(w), _f(tb), ctypes.byref(tl), _f(out), T, C, kernel)
    return out, tb[:max(kernel - 1, 0)], int(tl.value)


def available() -> bool:
    return kernels() is not None and transformer() is not None


def _f(a):
    if a is None:
        return ctypes.cast(None, POINTER(c_float))
    return a.ctypes.data_as(POINTER(c_float))


def _i(a):
    if a is None:
        return ctypes.cast(None, POINTER(c_int32))
    return a.ctypes.data_as(POINTER(c_int32))


def dequant(t: int, raw: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    out = np.zeros(n, dtype=np.float32)
    p = raw.ctypes.data_as(POINTER(c_uint8))
    if threads > 1:
        ok = kernels().aero_dequant_threaded(t, p, raw.size, _f(out), n, threads)
    else:
        ok = kernels().aero_dequant_ref(t, p, raw.size, _f(out), n)
    if not ok:
        raise ValueError("reference dequant refused")
    return out


def matvec(t: int, w: np.ndarray, x, n_rows: int, threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.zeros(n_rows, dtype=np.float32)
    if not kernels().aero_matvec(t, w.ctypes.data_as(POINTER(c_uint8)), _f(x), _f(y),
                                 n_rows, x.size, threads):
        raise ValueError("reference matvec refused")
    return y


def matmul(t: int, w: np.ndarray, X, n_rows: int, threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    X = np.ascontiguousarray(X, dtype=np.float32)
    T, n_cols = X.shape
    Y = np.zeros((T, n_rows), dtype=np.float32)
    if not kernels().aero_matmul(t, w.ctypes.data_as(POINTER(c_uint8)), _f(X), _f(Y), T,
                                 n_rows, n_cols, threads):
        raise ValueError("reference matmul refused")
    return Y


def rmsnorm_rows(x, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    transformer().aero_rmsnorm_rows(_f(x), _f(w), _f(out), x.size // cols, cols,
                                    float(eps))
    return out


def l2norm_rows(x, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    w = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    transformer().aero_l2norm_rows(_f(x), _f(w), _f(out), x.size // cols, cols,
                                   float(eps))
    return out


def act(name: str, x) -> np.ndarray:
    out = np.array(np.ascontiguousarray(x, dtype=np.float32), copy=True)
    getattr(transformer(), "aero_" + name)(_f(out), out.size)
    return out


def swiglu(g, u) -> np.ndarray:
    out = np.array(np.ascontiguousarray(g, dtype=np.float32), copy=True)
    u = np.ascontiguousarray(u, dtype=np.float32)
    transformer().aero_swiglu(_f(out), _f(u), out.size)
    return out


def mul(a, b) -> np.ndarray:
    out = np.array(np.ascontiguousarray(a, dtype=np.float32), copy=True)
    b = np.ascontiguousarray(b, dtype=np.float32)
    transformer().aero_tensor_mul(_f(out), _f(b), out.size)
    return out


def rope_tables(head_dim: int, positions, base: float, n_dims=None, ff=None):
    pos = np.ascontiguousarray(positions, dtype=np.int32).reshape(-1)
    n = head_dim if n_dims is None else min(int(n_dims), head_dim)
    n -= n % 2
    half = n // 2
    ffa = None if ff is None else np.ascontiguousarray(ff, dtype=np.float32)
    cos = np.zeros(max(pos.size * half, 1), dtype=np.float32)
    sin = np.zeros(max(pos.size * half, 1), dtype=np.float32)
    got = transformer().aero_rope_tables(head_dim, _i(pos), pos.size, float(base),
                                         -1 if n_dims is None else int(n_dims),
                                         _f(ffa), 0 if ffa is None else ffa.size,
                                         _f(cos), _f(sin))
    if got < 0:
        raise ValueError("reference rope_tables refused")
    h = got // 2
    return cos[: pos.size * h].reshape(pos.size, h), sin[: pos.size * h].reshape(pos.size, h)


def apply_rope(x, cos, sin, positions=None, mode: int = 0, n_rot=None) -> np.ndarray:
    out = np.array(np.ascontiguousarray(x, dtype=np.float32), copy=True)
    head_dim = out.shape[-1]
    cos = np.ascontiguousarray(cos, dtype=np.float32)
    sin = np.ascontiguousarray(sin, dtype=np.float32)
    n_rot = 2 * cos.shape[1] if n_rot is None else n_rot
    pos = None if positions is None else np.ascontiguousarray(positions, np.int32)
    transformer().aero_apply_rope(_f(out), out.size // head_dim, head_dim, n_rot,
                                  _f(cos), _f(sin), _i(pos), mode)
    return out


def dense_matmul(w, X, threads: int = 1) -> np.ndarray:
    """The reference's aero_tensor_matvec (one token) / aero_tensor_matmul."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    X = np.atleast_2d(np.ascontiguousarray(X, dtype=np.float32))
    Y = np.empty((X.shape[0], w.shape[0]), np.float32)
    L = transformer()
    if X.shape[0] == 1:
        ok = L.aero_tensor_matvec(_f(w), _f(X), _f(Y), w.shape[0], w.shape[1], threads)
    else:
        ok = L.aero_tensor_matmul(_f(w), _f(X), _f(Y), X.shape[0], w.shape[0], w.shape[1],
                                  threads)
    assert ok
    return Y


def argmax(v) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    return int(transformer().aero_tensor_argmax(_f(v), v.size))


def softmax(x) -> np.ndarray:
    out = np.array(np.ascontiguousarray(x, dtype=np.float32), copy=True)
    cols = out.shape[-1]
    transformer().aero_softmax_rows(_f(out), out.size // cols, cols)
    return out


def _i32(a):
    if a is None:
        return ctypes.cast(None, POINTER(c_int32))
    return a.ctypes.data_as(POINTER(c_int32))


def attention_tiled(q, k, v, scale: float, qpos=None, kpos=None, block: int = 1024,
                    window=None) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, H, D = q.shape
    S, HK, DV = k.shape[0], k.shape[1], v.shape[2]
    out = np.zeros((T, H, DV), np.float32)
    qp = None if qpos is None else np.ascontiguousarray(qpos, np.int32).reshape(-1)
    kp = None if kpos is None else np.ascontiguousarray(kpos, np.int32).reshape(-1)
    if not transformer().aero_attention_tiled(_f(q), _f(k), _f(v), _f(out), T, H, HK, D, DV,
                                              float(scale), _i32(qp), _i32(kp), S,
                                              0 if window is None else int(window), int(block)):
        raise ValueError("reference attention refused")
    return out


def kv_write_vec(dt: int, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    nbytes = {0: 4 * x.size, 1: x.size, 2: x.size // 2}[dt]
    q = np.zeros(nbytes, np.uint8)
    s = np.zeros(1, np.float32)
    if not kv().aero_kv_write_vec(dt, _f(x), x.size, q.ctypes.data, _f(s)):
        raise ValueError("reference kv write refused")
    return q, float(s[0])


def kv_span_error(dt: int, q, scale: float, x) -> float:
    q = np.ascontiguousarray(q, np.uint8)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    s = np.array([scale], np.float32)
    out = np.zeros(1, np.float32)
    if not kv().aero_kv_span_error(dt, q.ctypes.data, _f(s), x.size, _f(x), _f(out)):
        raise ValueError("reference kv span error refused")
    return float(out[0])


def kv_ring_rotate(cap: int, start: int, n: int):
    out = np.zeros(max(n, 1), np.int64)
    ok = kv().aero_kv_ring_rotate(cap, start, n, out.ctypes.data_as(POINTER(c_int64)))
    return ok, out[:n]


def kv_slot_roundtrip(cap: int, heads: int, dim: int, dt: int, writes):
    """The reference's KvSlot: write each (phys, head, x) of `writes`, then
    read every vector back; returns (bytes, [cap, heads, dim] fp32)."""
    L = kv()
    sl = L.aero_kv_slot_new(cap, heads, dim, dt, 0)
    assert sl
    try:
        for phys, head, x in writes:
            x = np.ascontiguousarray(x, np.float32)
            assert L.aero_kv_slot_write(sl, phys, head, _f(x))
        out = np.zeros((cap, heads, dim), np.float32)
        for p in range(cap):
            for h in range(heads):
                assert L.aero_kv_slot_read(sl, p, h, _f(out[p, h]))
        return int(L.aero_kv_slot_bytes(sl)), out
    finally:
        L.aero_kv_slot_free(sl)


def kv_read_vec(dt: int, q, scale: float, dim: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    s = np.array([scale], np.float32)
    out = np.zeros(dim, np.float32)
    if not kv().aero_kv_read_vec(dt, q.ctypes.data, _f(s), dim, _f(out)):
        raise ValueError("reference kv read refused")
    return out
