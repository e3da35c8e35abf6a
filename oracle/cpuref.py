"""ctypes binding of the oracle's C restatement (libaero_cpuref.so).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Every function takes and
returns numpy arrays; the C side follows the reference file:line cited in
oracle/cpuref.c and oracle/cpuref_quant.c.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint8, c_uint16

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaero_cpuref.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, BF16 = 0, 1, 8, 12, 13, 14, 23, 30
ACT_SILU, ACT_GELU, ACT_GELU_TANH, ACT_IDENTITY, ACT_SIGMOID = 0, 1, 2, 3, 4
ROPE_NEOX, ROPE_INTERLEAVED = 0, 1

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        fp, ip, up = POINTER(c_float), POINTER(c_int32), POINTER(c_uint8)
        L.cr_f16_to_f32.argtypes = [c_uint16]
        L.cr_f16_to_f32.restype = c_float
        L.cr_f16_to_f32_n.argtypes = [POINTER(c_uint16), fp, c_int64]
        L.cr_f16_to_f32_n.restype = None
        L.cr_block_bytes.argtypes = [c_int]
        L.cr_block_bytes.restype = c_int64
        L.cr_block_values.argtypes = [c_int]
        L.cr_block_values.restype = c_int64
        L.cr_dequant.argtypes = [c_int, up, c_int64, fp, c_int64]
        L.cr_dequant.restype = c_int
        L.cr_dequant_threaded.argtypes = [c_int, up, c_int64, fp, c_int64, c_int]
        L.cr_dequant_threaded.restype = c_int
        L.cr_matvec.argtypes = [c_int, up, fp, fp, c_int64, c_int64]
        L.cr_matvec.restype = c_int
        L.cr_matmul.argtypes = [c_int, up, fp, fp, c_int64, c_int64, c_int64]
        L.cr_matmul.restype = c_int
        L.cr_embed_gather.argtypes = [c_int, up, c_int64, c_int64, ip, c_int64,
                                      c_float, fp]
        L.cr_embed_gather.restype = c_int
        L.cr_rmsnorm_rows.argtypes = [fp, fp, fp, c_int64, c_int64, c_float, c_int]
        L.cr_rmsnorm_rows.restype = None
        L.cr_l2norm_rows.argtypes = [fp, fp, fp, c_int64, c_int64, c_float]
        L.cr_l2norm_rows.restype = None
        L.cr_gated_rmsnorm_silu.argtypes = [fp, fp, fp, c_int64, fp, c_int64,
                                            c_int64, c_int64, c_float]
        L.cr_gated_rmsnorm_silu.restype = None
        L.cr_act.argtypes = [c_int, fp, c_int64]
        L.cr_act.restype = None
        L.cr_act_mul.argtypes = [c_int, fp, fp, fp, c_int64]
        L.cr_act_mul.restype = None
        L.cr_rope_inv_freq.argtypes = [c_int64, c_int64, c_float, fp, c_int64, fp]
        L.cr_rope_inv_freq.restype = c_int64
        L.cr_rope_tables.argtypes = [c_int64, ip, c_int64, c_float, c_int64, fp,
                                     c_int64, fp, fp]
        L.cr_rope_tables.restype = c_int64
        L.cr_apply_rope.argtypes = [fp, c_int64, c_int64, c_int64, fp, fp, ip, c_int]
        L.cr_apply_rope.restype = None
        L.cr_dense_matvec.argtypes = [fp, fp, fp, c_int64, c_int64]
        L.cr_dense_matvec.restype = None
        L.cr_dense_matmul.argtypes = [fp, fp, fp, c_int64, c_int64, c_int64]
        L.cr_dense_matmul.restype = None
        L.cr_argmax.argtypes = [fp, c_int64]
        L.cr_argmax.restype = ctypes.c_int
        L.cr_softmax_rows.argtypes = [fp, c_int64, c_int64]
        L.cr_softmax_rows.restype = None
        L.cr_attention_tiled.argtypes = [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64,
                                         c_int64, c_float, ip, ip, c_int64, c_int, c_int64]
        L.cr_attention_tiled.restype = c_int
        L.cr_attention.argtypes = [fp, fp, fp, fp, c_int64, c_int64, c_int64, c_int64,
                                   c_float, c_int64, c_int]
        L.cr_attention.restype = c_int
        L.cr_kv_write_vec.argtypes = [c_int, fp, c_int64, ctypes.c_void_p, fp]
        L.cr_kv_write_vec.restype = c_int
        L.cr_kv_read_vec.argtypes = [c_int, ctypes.c_void_p, fp, c_int64, fp]
        L.cr_kv_read_vec.restype = c_int
        L.cr_ssm_softplus.argtypes = [c_float]
        L.cr_ssm_softplus.restype = c_float
        L.cr_ssm_delta_step_grouped.argtypes = [fp] * 8 + [c_int64] * 3 + [c_float, c_float, fp]
        L.cr_ssm_delta_step_grouped.restype = None
        L.cr_ssm_scan.argtypes = [fp] * 8 + [c_int64] * 4 + [c_float, c_float, fp]
        L.cr_ssm_scan.restype = None
        L.cr_ssm_conv.argtypes = [fp, fp, fp, POINTER(ctypes.c_int), fp, c_int64, c_int64,
                                  c_int64]
        L.cr_ssm_conv.restype = None
        _lib = L
    return _lib


def _f(a):
    if a is None:
        return ctypes.cast(None, POINTER(c_float))
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(POINTER(c_float))


def _i(a):
    if a is None:
        return ctypes.cast(None, POINTER(c_int32))
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(POINTER(c_int32))


def _u8(a):
    assert a.dtype == np.uint8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(POINTER(c_uint8))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def f16_to_f32(h: int) -> float:
    return float(lib().cr_f16_to_f32(int(h)))


def f16_bits_to_f32(h) -> np.ndarray:
    """Vector form (no Python-float round trip, so NaN payloads survive)."""
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(h.size, dtype=np.float32)
    lib().cr_f16_to_f32_n(h.ctypes.data_as(POINTER(c_uint16)), _f(out), h.size)
    return out


def block_bytes(t: int) -> int:
    return int(lib().cr_block_bytes(t))


def block_values(t: int) -> int:
    return int(lib().cr_block_values(t))


def dequant(t: int, raw: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    out = np.zeros(n, dtype=np.float32)
    if threads > 1:
        ok = lib().cr_dequant_threaded(t, _u8(raw), raw.size, _f(out), n, threads)
    else:
        ok = lib().cr_dequant(t, _u8(raw), raw.size, _f(out), n)
    if not ok:
        raise ValueError("oracle dequant refused")
    return out


def matvec(t: int, w: np.ndarray, x, n_rows: int) -> np.ndarray:
    """y = W @ x with W [n_rows, x.size] in quant blocks (src/kernels.cpp:497-515)."""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    x = f32(x).reshape(-1)
    y = np.zeros(n_rows, dtype=np.float32)
    if not lib().cr_matvec(t, _u8(w), _f(x), _f(y), n_rows, x.size):
        raise ValueError("oracle matvec refused")
    return y


def matmul(t: int, w: np.ndarray, X, n_rows: int) -> np.ndarray:
    """Y = X @ W^T, X [T, n_cols] (src/kernels.cpp:517-538)."""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1)
    X = f32(X)
    T, n_cols = X.shape
    Y = np.zeros((T, n_rows), dtype=np.float32)
    if not lib().cr_matmul(t, _u8(w), _f(X), _f(Y), T, n_rows, n_cols):
        raise ValueError("oracle matmul refused")
    return Y


def embed_gather(t: int, table: np.ndarray, vocab: int, n_embd: int, ids,
                 scale: float = 0.0) -> np.ndarray:
    table = np.ascontiguousarray(table, dtype=np.uint8).reshape(-1)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    out = np.zeros((ids.size, n_embd), dtype=np.float32)
    if not lib().cr_embed_gather(t, _u8(table), vocab, n_embd, _i(ids), ids.size,
                                 float(scale), _f(out)):
        raise ValueError("oracle embed_gather refused")
    return out


def rmsnorm_rows(x, w, eps: float, unit_offset: bool = False) -> np.ndarray:
    x = f32(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty_like(x)
    w = None if w is None else f32(w)
    lib().cr_rmsnorm_rows(_f(x), _f(w), _f(out), rows, cols, float(eps),
                          1 if unit_offset else 0)
    return out


def l2norm_rows(x, w, eps: float) -> np.ndarray:
    x = f32(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty_like(x)
    w = None if w is None else f32(w)
    lib().cr_l2norm_rows(_f(x), _f(w), _f(out), rows, cols, float(eps))
    return out


def gated_rmsnorm_silu(x, z, w, eps: float, group: int | None = None) -> np.ndarray:
    x, z, w = f32(x), f32(z), f32(w)
    inner = x.shape[-1]
    rows = x.size // inner
    group = inner if group is None else int(group)
    out = np.empty_like(x)
    lib().cr_gated_rmsnorm_silu(_f(x), _f(z), _f(w), w.size, _f(out), rows, inner,
                                group, float(eps))
    return out


def act(kind: int, x) -> np.ndarray:
    out = np.array(f32(x), copy=True)
    lib().cr_act(kind, _f(out), out.size)
    return out


def act_mul(kind: int, gate, up) -> np.ndarray:
    gate = f32(gate)
    up = None if up is None else f32(up)
    out = np.empty_like(gate)
    lib().cr_act_mul(kind, _f(gate), _f(up), _f(out), gate.size)
    return out


def rope_inv_freq(head_dim: int, n_dims, base: float, ff=None):
    ffa = None if ff is None else f32(ff).reshape(-1)
    inv = np.zeros(4096, dtype=np.float32)
    n = lib().cr_rope_inv_freq(head_dim, -1 if n_dims is None else int(n_dims),
                               float(base), _f(ffa), 0 if ffa is None else ffa.size,
                               _f(inv))
    if n < 0:
        raise ValueError("oracle rope_inv_freq refused")
    return int(n), inv[: n // 2].copy()


def rope_tables(head_dim: int, positions, base: float, n_dims=None, ff=None):
    pos = np.ascontiguousarray(positions, dtype=np.int32).reshape(-1)
    n = head_dim if n_dims is None else min(int(n_dims), head_dim)
    n -= n % 2
    half = n // 2
    ffa = None if ff is None else f32(ff).reshape(-1)
    cos = np.zeros(max(pos.size * half, 1), dtype=np.float32)
    sin = np.zeros(max(pos.size * half, 1), dtype=np.float32)
    got = lib().cr_rope_tables(head_dim, _i(pos), pos.size, float(base),
                               -1 if n_dims is None else int(n_dims), _f(ffa),
                               0 if ffa is None else ffa.size, _f(cos), _f(sin))
    if got < 0:
        raise ValueError("oracle rope_tables refused")
    h = got // 2
    return cos[: pos.size * h].reshape(pos.size, h), sin[: pos.size * h].reshape(pos.size, h)


def apply_rope(x, cos, sin, positions=None, mode: int = ROPE_NEOX,
               n_rot: int | None = None) -> np.ndarray:
    """Rotated copy of x (..., head_dim); table rows are read by positions[row]."""
    out = np.array(f32(x), copy=True)
    head_dim = out.shape[-1]
    rows = out.size // head_dim
    cos, sin = f32(cos), f32(sin)
    n_rot = 2 * cos.shape[1] if n_rot is None else n_rot
    pos = None if positions is None else np.ascontiguousarray(positions, np.int32)
    lib().cr_apply_rope(_f(out), rows, head_dim, n_rot, _f(cos), _f(sin), _i(pos), mode)
    return out


def qk_norm_rope(x, n_tok: int, n_head: int, head_dim: int, n_rot: int, pos,
                 base: float, mode: int = ROPE_NEOX, norm_w=None, eps: float = 1e-6,
                 unit_offset: bool = False, ff=None, cos_tab=None, sin_tab=None):
    """The composition the fused kernel reproduces (src/attention_layer.cpp:89-156):
    optional per-(token, head) RMSNorm over head_dim, then RoPE on the first
    n_rot channels at the token's position. Angles come from a table built by
    rope_tables over the token positions (row t <-> token t), or, when cos_tab /
    sin_tab are given, from that POSITION-indexed table."""
    x = f32(x).reshape(n_tok, n_head, head_dim)
    pos = np.ascontiguousarray(pos, dtype=np.int32).reshape(-1)
    if norm_w is not None:
        x = rmsnorm_rows(x, norm_w, eps, unit_offset)
    if n_rot < 2:
        return np.array(x, copy=True)
    if cos_tab is None:
        c, s = rope_tables(n_rot, pos, base, n_rot, ff)
        rowpos = np.repeat(np.arange(n_tok, dtype=np.int32), n_head)
    else:
        c, s = cos_tab, sin_tab
        rowpos = np.repeat(pos, n_head)
    return apply_rope(x, c, s, rowpos, mode, n_rot=n_rot)


# ------------------------------------------------------- softmax, attention
def dense_matvec(w, x) -> np.ndarray:
    """src/tensor.cpp:65-81: y = W x, fp32, four products at a time."""
    w = f32(w)
    x = f32(x).reshape(-1)
    y = np.empty(w.shape[0], np.float32)
    lib().cr_dense_matvec(_f(w), _f(x), _f(y), w.shape[0], w.shape[1])
    return y


def dense_matmul(w, X) -> np.ndarray:
    """src/tensor.cpp:83-92: Y = X W^T, fp32."""
    w = f32(w)
    X = np.atleast_2d(f32(X))
    Y = np.empty((X.shape[0], w.shape[0]), np.float32)
    lib().cr_dense_matmul(_f(w), _f(X), _f(Y), X.shape[0], w.shape[0], w.shape[1])
    return Y


def argmax(v) -> int:
    """src/tensor.cpp:180-186: first index of the largest value (strict '>'
    scan from v[0])."""
    v = f32(v).reshape(-1)
    return int(lib().cr_argmax(_f(v), v.size))


def softmax(x) -> np.ndarray:
    """src/tensor.cpp:167-178 over the last axis."""
    out = np.array(f32(x), copy=True)
    cols = out.shape[-1] if out.ndim else 1
    lib().cr_softmax_rows(_f(out), out.size // max(cols, 1), cols)
    return out


def attention_tiled(q, k, v, scale: float, qpos=None, kpos=None, block: int = 1024,
                    window=None) -> np.ndarray:
    """src/transformer.cpp:120-203. q (T,H,D), k (S,HK,D), v (S,HK,DV) -> (T,H,DV)."""
    q, k, v = f32(q), f32(k), f32(v)
    T, H, D = q.shape
    S, HK, DV = k.shape[0], k.shape[1], v.shape[2]
    out = np.zeros((T, H, DV), np.float32)
    qp = None if qpos is None else np.ascontiguousarray(qpos, np.int32).reshape(-1)
    kp = None if kpos is None else np.ascontiguousarray(kpos, np.int32).reshape(-1)
    ok = lib().cr_attention_tiled(_f(q), _f(k), _f(v), _f(out), T, H, HK, D, DV, float(scale),
                                  _i(qp), _i(kp), S, 0 if window is None else int(window),
                                  int(block))
    if not ok:
        raise ValueError("attention refused")
    return out


def attention(q, k, v, scale: float, window=None) -> np.ndarray:
    """src/transformer.cpp:205-214: one query at position S-1. q (H,D)."""
    q, k, v = f32(q), f32(k), f32(v)
    H, D = q.shape
    S, HK, DV = k.shape[0], k.shape[1], v.shape[2]
    out = np.zeros((H, DV), np.float32)
    ok = lib().cr_attention(_f(q), _f(k), _f(v), _f(out), H, HK, D, DV, float(scale), S,
                            0 if window is None else int(window))
    if not ok:
        raise ValueError("attention refused")
    return out


KV_F32, KV_I8, KV_I4 = 0, 1, 2


def kv_write_vec(dt: int, x):
    """src/kv.cpp:13-26: (packed vector as uint8 bytes, scale)."""
    x = f32(x).reshape(-1)
    nbytes = {KV_F32: 4 * x.size, KV_I8: x.size, KV_I4: x.size // 2}[dt]
    q = np.zeros(nbytes, np.uint8)
    s = np.zeros(1, np.float32)
    if not lib().cr_kv_write_vec(dt, _f(x), x.size, q.ctypes.data, _f(s)):
        raise ValueError("kv write refused")
    return q, float(s[0])


def kv_read_vec(dt: int, q, scale: float, dim: int) -> np.ndarray:
    """src/kv.cpp:29-46."""
    q = np.ascontiguousarray(q, np.uint8)
    s = np.array([scale], np.float32)
    out = np.zeros(dim, np.float32)
    if not lib().cr_kv_read_vec(dt, q.ctypes.data, _f(s), dim, _f(out)):
        raise ValueError("kv read refused")
    return out


# ------------------------------------------------------------ gated DeltaNet

def ssm_softplus(x) -> np.ndarray:
    """src/ssm.cpp:22-24, elementwise."""
    x = f32(x)
    return np.array([lib().cr_ssm_softplus(float(v)) for v in x.reshape(-1)],
                    np.float32).reshape(x.shape)


def ssm_delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """src/ssm.cpp:69-126. q, k (n_k, d); v (n_v, d); state (n_v, d, d), not
    mutated. Returns (out (n_v, d), new state)."""
    q, k, v = f32(q), f32(k), f32(v)
    n_k, d = q.shape
    n_v = v.shape[0]
    st = np.array(f32(state), copy=True)
    out = np.zeros((n_v, d), np.float32)
    lib().cr_ssm_delta_step_grouped(_f(q), _f(k), _f(v), _f(f32(alpha)), _f(f32(beta)),
                                    _f(f32(a_log)), _f(f32(dt_bias)), _f(st), n_k, n_v, d,
                                    float(scale), float(eps), _f(out))
    return out, st


def ssm_scan(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """src/ssm.cpp:128-142,163-171. q, k (T, n_k, d); v (T, n_v, d); alpha,
    beta (T, n_v). Returns (outs (T, n_v, d), new state)."""
    q, k, v = f32(q), f32(k), f32(v)
    T, n_k, d = q.shape
    n_v = v.shape[1]
    st = np.array(f32(state), copy=True)
    outs = np.zeros((T, n_v, d), np.float32)
    lib().cr_ssm_scan(_f(q), _f(k), _f(v), _f(f32(alpha)), _f(f32(beta)), _f(f32(a_log)),
                      _f(f32(dt_bias)), _f(st), T, n_k, n_v, d, float(scale), float(eps),
                      _f(outs))
    return outs, st


def ssm_forward(x, dts, weights, a_log, dt_bias, conv1d, norm, n_k: int, d: int, inner: int,
                eps: float, norm_eps: float, tail, tail_len: int, state):
    """One gated-DeltaNet layer, aero_ssm_forward_q (src/ssm.cpp:262-352),
    composed from the oracle's restatements. x [T, n_embd] is the layer's
    (already normed) input; dts / weights list the (qkv, gate, alpha, beta,
    out) projections (:224-225), each [n_out, n_in]: dtype 0 a float32 array,
    else raw GGUF blocks; conv1d [qkv, K] with qkv = 2 n_k d + inner; norm [d]
    tiled over the n_v = inner / d heads; tail [K-1, qkv] holds tail_len rows
    of conv history; state [n_v, d, d]. Returns (out [T, n_embd], tail,
    tail_len, state), the inputs untouched.
    - :289-296 the qkv projection per token, then (:297) the causal conv over
      [tail; qkv] and (:298-301) silu = x / (1 + exp(-x)) on every element;
    - :303-315 alpha, beta (n_v each) and gate (inner) from x;
    - :316-320 the scan over the q / k / v slices of each qkv row, scale
      1/sqrt(d), the l2 eps eps;
    - :322-340 the gated RMSNorm over the whole row (group = inner), norm eps
      norm_eps, w[c % d];
    - :343-348 the output projection.
    float32 projections are evaluated in float64 and rounded (the reference
    sums them serially in float32: matvec_fp32, :37-44)."""
    x = f32(x)
    T, n_embd = x.shape
    n_v = inner // d
    qkv_w = 2 * n_k * d + inner

    def proj(i, X, n_out):
        if dts[i] == F32:
            W = np.asarray(weights[i], np.float32).reshape(n_out, X.shape[1])
            return (X.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32)
        return matmul(dts[i], weights[i], X, n_out)

    qkv = proj(0, x, qkv_w)
    conv, tail2, tl2 = ssm_conv(qkv, conv1d, tail, tail_len)
    conv = conv / (np.float32(1.0) + np.exp(-conv))
    alpha = proj(2, x, n_v)
    beta = proj(3, x, n_v)
    gate = proj(1, x, inner)
    q = conv[:, :n_k * d].reshape(T, n_k, d)
    k = conv[:, n_k * d:2 * n_k * d].reshape(T, n_k, d)
    v = conv[:, 2 * n_k * d:].reshape(T, n_v, d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    outs, st = ssm_scan(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps)
    o = gated_rmsnorm_silu(outs.reshape(T, inner), gate, norm, norm_eps, group=inner)
    return proj(4, o, n_embd), tail2, tl2, st


def ssm_conv(x, w, tail, tail_len: int):
    """src/ssm.cpp:173-210. x (T, C); w (C, kernel); tail (>= kernel-1, C)
    holding tail_len rows. Returns (out, new tail (kernel-1, C), new length)."""
    x, w = f32(x), f32(w)
    T, C = x.shape
    kernel = w.shape[1]
    tb = np.zeros((max(kernel - 1, 1), C), np.float32)
    if tail_len > 0:
        tb[:tail_len] = f32(tail)[:tail_len]
    out = np.zeros((T, C), np.float32)
    tl = ctypes.c_int(int(tail_len))
    lib().cr_ssm_conv(_f(x), _f(w), _f(tb), ctypes.byref(tl), _f(out), T, C, kernel)
    return out, tb[:max(kernel - 1, 0)], int(tl.value)
