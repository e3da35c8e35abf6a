"""Device-resident fused ops: the aero_hip_* entry points over DeviceArrays.

Every function checks on the host that each buffer is large enough for the
shape it is given before anything is launched, then enqueues one kernel on
`stream` (None = the null stream) and returns without waiting. These are the
ops a model loop calls with activations already in HBM; the reference-shaped
numpy wrappers live in tensor_native / transformer_native / native.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceArray, Stream, Workspace, as_ptr

NORM_UNIT_OFFSET = 1
NORM_L2 = 2

ACT_SILU = 0
ACT_GELU = 1
ACT_GELU_TANH = 2
ACT_IDENTITY = 3
ACT_SIGMOID = 4
ACTS = {"silu": ACT_SILU, "swiglu": ACT_SILU, "gelu": ACT_GELU, "geglu": ACT_GELU,
        "gelu_erf": ACT_GELU, "gelu_tanh": ACT_GELU_TANH, "geglu_tanh": ACT_GELU_TANH,
        "identity": ACT_IDENTITY, "mul": ACT_IDENTITY, "sigmoid": ACT_SIGMOID}

ROPE_NEOX = 0
ROPE_INTERLEAVED = 1

DTYPE_F32, DTYPE_F16, DTYPE_Q8_0, DTYPE_Q4_K, DTYPE_Q6_K, DTYPE_BF16 = 0, 1, 8, 12, 14, 30
DTYPE_Q5_K, DTYPE_IQ4_XS = 13, 23
_BLOCK = {DTYPE_F32: (1, 4), DTYPE_F16: (1, 2), DTYPE_BF16: (1, 2), DTYPE_Q8_0: (32, 34),
          DTYPE_Q4_K: (256, 144), DTYPE_Q5_K: (256, 176), DTYPE_Q6_K: (256, 210),
          DTYPE_IQ4_XS: (256, 136)}


def _s(stream: Stream | None):
    return None if stream is None else stream.handle


def _need(arr, nelem: int, dtype, name: str):
    if arr is None:
        return
    if not isinstance(arr, DeviceArray):
        raise TypeError(f"{name}: expected a DeviceArray, got {type(arr).__name__}")
    if arr.dtype != np.dtype(dtype):
        raise TypeError(f"{name}: dtype {arr.dtype}, expected {np.dtype(dtype)}")
    if arr.size < nelem:
        raise ValueError(f"{name}: holds {arr.size} elements, needs {nelem}")


def rmsnorm(x: DeviceArray, w: DeviceArray | None, out: DeviceArray, rows: int, cols: int,
            eps: float, unit_offset: bool = False, l2: bool = False,
            stream: Stream | None = None) -> None:
    """out[r] = x[r]/sqrt(mean(x[r]^2)+eps) * (w or 1+w); L2 form with l2=True."""
    _need(x, rows * cols, np.float32, "x")
    _need(out, rows * cols, np.float32, "out")
    _need(w, cols, np.float32, "w")
    flags = (NORM_UNIT_OFFSET if unit_offset else 0) | (NORM_L2 if l2 else 0)
    L = _lib.lib()
    _lib.check(L.aero_hip_rmsnorm(x.ptr, as_ptr(w), out.ptr, rows, cols, float(eps), flags,
                                  _s(stream)), "rmsnorm")


def gated_rmsnorm_silu(x: DeviceArray, z: DeviceArray, w: DeviceArray, out: DeviceArray,
                       rows: int, inner: int, eps: float, group: int | None = None,
                       stream: Stream | None = None) -> None:
    """out = rmsnorm_group(x) * tile(w) * silu(z); group=None is the whole row."""
    group = inner if group is None else int(group)
    _need(x, rows * inner, np.float32, "x")
    _need(z, rows * inner, np.float32, "z")
    _need(out, rows * inner, np.float32, "out")
    _need(w, 1, np.float32, "w")
    _lib.check(_lib.lib().aero_hip_gated_rmsnorm_silu(x.ptr, z.ptr, w.ptr, w.size, out.ptr,
                                                      rows, inner, group, float(eps),
                                                      _s(stream)), "gated_rmsnorm_silu")


def post_norm_add(y: DeviceArray, x: DeviceArray, w_post: DeviceArray | None,
                  w_next: DeviceArray | None, h: DeviceArray, rows: int, cols: int, eps: float,
                  ds: float = 1.0, ss: float = 1.0, unit_offset: bool = False,
                  x_out: DeviceArray | None = None, stream: Stream | None = None) -> None:
    """A Gemma sandwich-norm site in one pass: x_out = (x + ds * rmsnorm(y) *
    w_post) * ss (x_out None: x in place), h = rmsnorm(x_out) * w_next."""
    x_out = x if x_out is None else x_out
    for a, name in ((y, "y"), (x, "x"), (x_out, "x_out"), (h, "h")):
        _need(a, rows * cols, np.float32, name)
    _need(w_post, cols, np.float32, "w_post")
    _need(w_next, cols, np.float32, "w_next")
    _lib.check(_lib.lib().aero_hip_post_norm_add(
        y.ptr, x.ptr, x_out.ptr, as_ptr(w_post), float(ds), float(ss), as_ptr(w_next), h.ptr,
        rows, cols, float(eps), NORM_UNIT_OFFSET if unit_offset else 0, _s(stream)),
        "post_norm_add")


def add_rmsnorm(x: DeviceArray, d: DeviceArray, w: DeviceArray | None, h: DeviceArray,
                rows: int, cols: int, eps: float, unit_offset: bool = False,
                x_out: DeviceArray | None = None, stream: Stream | None = None) -> None:
    """Residual add then RMSNorm in one pass: x_out = x + d (x_out None: x
    in place), h = rmsnorm(x_out) * (w or 1+w)."""
    x_out = x if x_out is None else x_out
    for a, name in ((x, "x"), (d, "d"), (x_out, "x_out"), (h, "h")):
        _need(a, rows * cols, np.float32, name)
    _need(w, cols, np.float32, "w")
    _lib.check(_lib.lib().aero_hip_add_rmsnorm(x.ptr, d.ptr, x_out.ptr, as_ptr(w), h.ptr, rows,
                                               cols, float(eps),
                                               NORM_UNIT_OFFSET if unit_offset else 0,
                                               _s(stream)), "add_rmsnorm")


def act_mul(kind, gate: DeviceArray, up: DeviceArray | None, out: DeviceArray,
            n: int | None = None, stream: Stream | None = None) -> None:
    """out = act(gate) * up (up None: out = act(gate)). kind: int or name."""
    k = ACTS[kind] if isinstance(kind, str) else int(kind)
    n = gate.size if n is None else int(n)
    _need(gate, n, np.float32, "gate")
    _need(up, n, np.float32, "up")
    _need(out, n, np.float32, "out")
    _lib.check(_lib.lib().aero_hip_act_mul(k, gate.ptr, as_ptr(up), out.ptr, n, _s(stream)),
               "act_mul")


def rope_inv_freq(head_dim: int, n_dims: int | None, base: float, freq_factors=None):
    """(n_rot, inv[n_rot/2]) on the host, bit-identical to the reference's."""
    import ctypes
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32).reshape(-1)
    inv = np.zeros(max(head_dim // 2, 1), dtype=np.float32)
    n = _lib.load().aero_hip_rope_inv_freq(
        head_dim, -1 if n_dims is None else int(n_dims), float(base),
        None if ff is None else ff.ctypes.data_as(_lib.fp), 0 if ff is None else ff.size,
        inv.ctypes.data_as(_lib.fp))
    if n < 0:
        raise ValueError(f"rope_inv_freq refused: {_lib.last_error()}")
    return int(n), inv[: n // 2].copy()


def rope_tables(pos: DeviceArray, inv: DeviceArray, cos_out: DeviceArray, sin_out: DeviceArray,
                stream: Stream | None = None) -> None:
    half = inv.size
    _need(pos, pos.size, np.int32, "pos")
    _need(cos_out, pos.size * half, np.float32, "cos")
    _need(sin_out, pos.size * half, np.float32, "sin")
    _lib.check(_lib.lib().aero_hip_rope_tables(pos.ptr, pos.size, inv.ptr, half, cos_out.ptr,
                                               sin_out.ptr, _s(stream)), "rope_tables")


def qk_norm_rope(q: DeviceArray, n_q_heads: int, n_tok: int, head_dim: int, n_rot: int,
                 *, k: DeviceArray | None = None, n_k_heads: int = 0,
                 q_out: DeviceArray | None = None, k_out: DeviceArray | None = None,
                 q_norm_w: DeviceArray | None = None, k_norm_w: DeviceArray | None = None,
                 eps: float = 1e-6, unit_offset: bool = False, mode: int = ROPE_NEOX,
                 pos: DeviceArray | None = None, inv_freq: DeviceArray | None = None,
                 cos_tab: DeviceArray | None = None, sin_tab: DeviceArray | None = None,
                 stream: Stream | None = None) -> None:
    """Per-head RMSNorm (optional) then RoPE on q [n_tok, Hq, D] and k [n_tok, Hk, D].
    Angles from inv_freq (computed) or a position-indexed cos/sin table."""
    half = n_rot // 2
    _need(q, n_tok * n_q_heads * head_dim, np.float32, "q")
    _need(q_out, n_tok * n_q_heads * head_dim, np.float32, "q_out")
    if n_k_heads:
        _need(k, n_tok * n_k_heads * head_dim, np.float32, "k")
        _need(k_out, n_tok * n_k_heads * head_dim, np.float32, "k_out")
        if k is None:
            raise ValueError("k is required when n_k_heads > 0")
    _need(q_norm_w, head_dim, np.float32, "q_norm_w")
    _need(k_norm_w, head_dim, np.float32, "k_norm_w")
    _need(pos, n_tok, np.int32, "pos")
    _need(inv_freq, half, np.float32, "inv_freq")
    n_tab = 0
    if cos_tab is not None or sin_tab is not None:
        if cos_tab is None or sin_tab is None or half == 0:
            raise ValueError("a table needs both cos_tab and sin_tab")
        n_tab = min(cos_tab.size, sin_tab.size) // half
        _need(cos_tab, n_tab * half, np.float32, "cos_tab")
        _need(sin_tab, n_tab * half, np.float32, "sin_tab")
    flags = NORM_UNIT_OFFSET if unit_offset else 0
    _lib.check(_lib.lib().aero_hip_qk_norm_rope(
        q.ptr, as_ptr(q_out), n_q_heads, as_ptr(k), as_ptr(k_out), n_k_heads,
        as_ptr(q_norm_w), as_ptr(k_norm_w), float(eps), flags, n_tok, head_dim, n_rot,
        int(mode), as_ptr(pos), as_ptr(inv_freq), as_ptr(cos_tab), as_ptr(sin_tab), n_tab,
        _s(stream)), "qk_norm_rope")


def row_bytes(dtype: int, n_embd: int) -> int:
    bv, bb = _BLOCK[dtype]
    if n_embd % bv:
        raise ValueError(f"n_embd {n_embd} is not a multiple of the block size {bv}")
    return (n_embd // bv) * bb


def embed_gather(dtype: int, table: DeviceArray, vocab: int, n_embd: int, ids: DeviceArray,
                 out: DeviceArray, scale: float = 0.0, bad_count: DeviceArray | None = None,
                 n_ids: int | None = None, stream: Stream | None = None) -> None:
    """out[i] = dequant(table row ids[i]) (* scale when scale > 0)."""
    n_ids = ids.size if n_ids is None else int(n_ids)
    rb = row_bytes(dtype, n_embd)
    if table.nbytes < vocab * rb:
        raise ValueError(f"table holds {table.nbytes} B, needs {vocab * rb}")
    _need(ids, n_ids, np.int32, "ids")
    _need(out, n_ids * n_embd, np.float32, "out")
    _need(bad_count, 1, np.uint32, "bad_count")
    _lib.check(_lib.lib().aero_hip_embed_gather(int(dtype), table.ptr, table.nbytes, vocab,
                                                n_embd, ids.ptr, n_ids, float(scale), out.ptr,
                                                as_ptr(bad_count), _s(stream)), "embed_gather")


def embed_rmsnorm(dtype: int, table: DeviceArray, vocab: int, n_embd: int, ids: DeviceArray,
                  x_out: DeviceArray, h_out: DeviceArray, norm_w: DeviceArray | None,
                  eps: float, scale: float = 0.0, unit_offset: bool = False,
                  bad_count: DeviceArray | None = None, n_ids: int | None = None,
                  stream: Stream | None = None) -> None:
    """Embedding gather and the first RMSNorm in one pass: x_out as
    embed_gather, h_out = rmsnorm(x_out) * (norm_w or 1+norm_w)."""
    n_ids = ids.size if n_ids is None else int(n_ids)
    rb = row_bytes(dtype, n_embd)
    if table.nbytes < vocab * rb:
        raise ValueError(f"table holds {table.nbytes} B, needs {vocab * rb}")
    _need(ids, n_ids, np.int32, "ids")
    _need(x_out, n_ids * n_embd, np.float32, "x_out")
    _need(h_out, n_ids * n_embd, np.float32, "h_out")
    _need(norm_w, n_embd, np.float32, "norm_w")
    _need(bad_count, 1, np.uint32, "bad_count")
    _lib.check(_lib.lib().aero_hip_embed_rmsnorm(
        int(dtype), table.ptr, table.nbytes, vocab, n_embd, ids.ptr, n_ids, float(scale),
        x_out.ptr, as_ptr(norm_w), float(eps), NORM_UNIT_OFFSET if unit_offset else 0,
        h_out.ptr, as_ptr(bad_count), _s(stream)), "embed_rmsnorm")


def dequant(dtype: int, raw: DeviceArray, out: DeviceArray, n_values: int,
            stream: Stream | None = None) -> None:
    bv, bb = _BLOCK[dtype]
    if raw.nbytes < (n_values // bv) * bb:
        raise ValueError("raw buffer too short")
    _need(out, (n_values // bv) * bv, np.float32, "out")
    _lib.check(_lib.lib().aero_hip_dequant(int(dtype), raw.ptr, raw.nbytes, out.ptr, n_values,
                                           _s(stream)), "dequant")


_gemm_ws = Workspace("split GEMM")


def split_ok(dtype: int, n_cols: int, n_rows: int, n_tok: int) -> bool:
    """True when a (norm_)matmul of this shape takes the split-x GEMM, the
    path whose pre-pass folds a residual add and an RMSNorm."""
    L = _lib.load()
    if L is None:
        raise _lib.AeroHipUnavailable(_lib.unavailable_reason())
    return bool(L.aero_hip_split_ok(int(dtype), int(n_cols), int(n_rows), int(n_tok)))


def matvec(dtype: int, w: DeviceArray, x: DeviceArray, y: DeviceArray, n_rows: int,
           n_cols: int, n_tok: int = 1, stream: Stream | None = None,
           split: bool = True) -> None:
    """y[t, r] = sum_c W[r, c] * x[t, c] for t < n_tok: W n_rows rows of quant
    blocks (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS), x [n_tok, n_cols], y [n_tok, n_rows].
    From 5-16 tokens (by matrix size), Q4_K, Q5_K, Q8_0, Q6_K (rows of 2048k
    columns) and IQ4_XS (512k) run the split-x fp16 matrix-core GEMM with a
    cached workspace (split=False: the fp32 matrix-core GEMM)."""
    if dtype not in _BLOCK or _BLOCK[dtype][0] == 1:
        raise ValueError(f"dtype {dtype} has no quantised GEMV")
    bv, bb = _BLOCK[dtype]
    if n_cols <= 0 or n_cols % bv:
        raise ValueError(f"n_cols {n_cols} must be a positive multiple of {bv}")
    if w.nbytes < n_rows * (n_cols // bv) * bb:
        raise ValueError("weight buffer too short")
    _need(x, n_tok * n_cols, np.float32, "x")
    _need(y, n_tok * n_rows, np.float32, "y")
    L = _lib.lib()
    wsb = int(L.aero_hip_matmul_workspace(int(dtype), n_cols, n_tok)) if n_tok > 1 else 0
    if wsb:      # room for column-split partials (few tokens)
        wsb += int(L.aero_hip_split_partials_bytes(n_rows, n_cols, n_tok))
    if wsb and split:
        ws = _gemm_ws.get(wsb)
        _lib.check(L.aero_hip_matmul(int(dtype), w.ptr, w.nbytes, x.ptr, y.ptr, n_rows, n_cols,
                                     n_tok, ws.ptr, ws.nbytes, _s(stream)), "matmul")
        return
    _lib.check(L.aero_hip_matvec(int(dtype), w.ptr, w.nbytes, x.ptr, y.ptr, n_rows,
                                 n_cols, n_tok, _s(stream)), "matvec")


def norm_matvec(dtype: int, ws: list, x: DeviceArray, ys: list, n_rows: list, n_cols: int,
                n_tok: int = 1, norm_w: DeviceArray | None = None, eps: float = 1e-5,
                norm: bool = True, unit_offset: bool = False,
                stream: Stream | None = None) -> None:
    """ys[m] = rmsnorm(x) @ W_m^T for up to 4 matrices of one type sharing x
    (q, k, v), in one launch per 4 tokens; norm=False uses x as is."""
    if not 1 <= len(ws) <= 4 or len(ys) != len(ws) or len(n_rows) != len(ws):
        raise ValueError("norm_matvec: 1 to 4 matrices, with as many outputs and row counts")
    _need(x, n_tok * n_cols, np.float32, "x")
    _need(norm_w, n_cols, np.float32, "norm_w")
    for y, nr in zip(ys, n_rows):
        _need(y, n_tok * nr, np.float32, "y")
    k = len(ws)
    wp = (ctypes.c_void_p * k)(*[w.ptr for w in ws])
    wb = (ctypes.c_int64 * k)(*[w.nbytes for w in ws])
    nr = (ctypes.c_int64 * k)(*[int(n) for n in n_rows])
    yp = (ctypes.c_void_p * k)(*[y.ptr for y in ys])
    flag = (NORM_UNIT_OFFSET if unit_offset else 0) if norm else -1
    _lib.check(_lib.lib().aero_hip_norm_matvec(int(dtype), k, wp, wb, nr, yp, x.ptr,
                                               as_ptr(norm_w), float(eps), flag, n_cols, n_tok,
                                               _s(stream)), "norm_matvec")


def norm_gate_up(dtype: int, w_gate: DeviceArray, w_up: DeviceArray, x: DeviceArray,
                 out: DeviceArray, n_ff: int, n_cols: int, n_tok: int = 1, act="silu",
                 norm_w: DeviceArray | None = None, eps: float = 1e-5, norm: bool = True,
                 unit_offset: bool = False, stream: Stream | None = None) -> None:
    """out = act(rmsnorm(x) @ Wg^T) * (rmsnorm(x) @ Wu^T) in one launch per 4
    tokens (SwiGLU / GeGLU decode); norm=False uses x as is."""
    kind = ACTS[act] if isinstance(act, str) else int(act)
    _need(x, n_tok * n_cols, np.float32, "x")
    _need(out, n_tok * n_ff, np.float32, "out")
    _need(norm_w, n_cols, np.float32, "norm_w")
    if w_gate.nbytes != w_up.nbytes:
        raise ValueError("norm_gate_up: gate and up must be the same size")
    flag = (NORM_UNIT_OFFSET if unit_offset else 0) if norm else -1
    _lib.check(_lib.lib().aero_hip_norm_gate_up(int(dtype), w_gate.ptr, w_up.ptr, w_gate.nbytes,
                                                x.ptr, as_ptr(norm_w), float(eps), flag, kind,
                                                out.ptr, n_ff, n_cols, n_tok, _s(stream)),
               "norm_gate_up")


_norm_mm_ws = Workspace("norm GEMM")


def ssm_proj_conv(dtype: int, ws: list, x: DeviceArray, ys: list, n_rows: list, n_cols: int,
                  conv_w: DeviceArray, tail: DeviceArray, tail_len: int, conv_out: DeviceArray,
                  stream: Stream | None = None) -> int:
    """One token of a DeltaNet layer's input projections (up to 4 matrices of
    one type sharing x) with matrix 0's rows (qkv) through the causal conv of
    kernel 4 and silu into conv_out, the history tail [3, n_rows[0]] moved on
    in place (src/ssm.cpp:289-315,297-301); ys[0] is not written. Returns the
    history's new length."""
    k = len(ws)
    if not 1 <= k <= 4 or len(ys) != k or len(n_rows) != k:
        raise ValueError("ssm_proj_conv: 1-4 matrices, one output and row count each")
    C = int(n_rows[0])
    _need(x, n_cols, np.float32, "x")
    _need(conv_w, 4 * C, np.float32, "conv_w")
    _need(tail, 3 * C, np.float32, "tail")
    _need(conv_out, C, np.float32, "conv_out")
    for y, n in zip(ys, n_rows):
        _need(y, int(n), np.float32, "y")
    wp = (ctypes.c_void_p * k)(*[w.ptr for w in ws])
    wb = (ctypes.c_int64 * k)(*[w.nbytes for w in ws])
    nr = (ctypes.c_int64 * k)(*[int(n) for n in n_rows])
    yp = (ctypes.c_void_p * k)(*[y.ptr for y in ys])
    _lib.check(_lib.lib().aero_hip_ssm_proj_conv(int(dtype), k, wp, wb, nr, yp, x.ptr, n_cols,
                                                 conv_w.ptr, tail.ptr, int(tail_len),
                                                 conv_out.ptr, _s(stream)), "ssm_proj_conv")
    return min(3, int(tail_len) + 1)


def gated_norm_matvec(dtype: int, w: DeviceArray, x: DeviceArray, z: DeviceArray,
                      norm_w: DeviceArray, y: DeviceArray, n_rows: int, n_cols: int,
                      n_tok: int, eps: float, stream: Stream | None = None) -> None:
    """y = gated_rmsnorm_silu(x, z, tile(norm_w)) @ W^T over whole rows, the
    norm in the GEMV's prologue (src/ssm.cpp:322-348, a DeltaNet layer's
    gated norm and output projection); up to 2 tokens."""
    _need(x, n_tok * n_cols, np.float32, "x")
    _need(z, n_tok * n_cols, np.float32, "z")
    _need(y, n_tok * n_rows, np.float32, "y")
    _need(norm_w, 1, np.float32, "norm_w")
    _lib.check(_lib.lib().aero_hip_gated_norm_matvec(int(dtype), w.ptr, w.nbytes, n_rows, y.ptr,
                                                     x.ptr, z.ptr, norm_w.ptr, norm_w.size,
                                                     float(eps), n_cols, n_tok, _s(stream)),
               "gated_norm_matvec")


def gated_norm_matmul(dtype: int, w: DeviceArray, x: DeviceArray, z: DeviceArray,
                      norm_w: DeviceArray, y: DeviceArray, n_rows: int, n_cols: int,
                      n_tok: int, eps: float, stream: Stream | None = None) -> None:
    """y = gated_rmsnorm_silu(x, z, tile(norm_w)) @ W^T over whole rows, any
    token count (src/ssm.cpp:322-348): the norm in the fused GEMV's prologue
    up to 2 tokens, in the split GEMM's x pre-pass on its path, else a gated
    norm pass into the workspace before the projection."""
    _need(x, n_tok * n_cols, np.float32, "x")
    _need(z, n_tok * n_cols, np.float32, "z")
    _need(y, n_tok * n_rows, np.float32, "y")
    _need(norm_w, 1, np.float32, "norm_w")
    L = _lib.lib()
    wsb = L.aero_hip_norm_matmul_workspace(int(dtype), n_cols, 0, n_tok)
    wsb += L.aero_hip_split_partials_bytes(int(n_rows), n_cols, n_tok)
    buf = _norm_mm_ws.get(wsb)
    _lib.check(L.aero_hip_gated_norm_matmul(int(dtype), w.ptr, w.nbytes, n_rows, y.ptr, x.ptr,
                                            z.ptr, norm_w.ptr, norm_w.size, float(eps), n_cols,
                                            n_tok, as_ptr(buf), 0 if buf is None else buf.nbytes,
                                            _s(stream)), "gated_norm_matmul")


def _norm_flag(norm: bool, unit_offset: bool) -> int:
    return (NORM_UNIT_OFFSET if unit_offset else 0) if norm else -1


def norm_matmul(dtype: int, ws: list, x: DeviceArray, ys: list, n_rows: list, n_cols: int,
                n_tok: int, norm_w: DeviceArray | None = None, eps: float = 1e-5,
                norm: bool = True, unit_offset: bool = False, d: DeviceArray | None = None,
                x_out: DeviceArray | None = None, rope: dict | None = None,
                stream: Stream | None = None) -> None:
    """ys[m] = rmsnorm(x') @ W_m^T for up to 4 matrices of one type sharing x'
    (q, k, v), any token count; x' = x + d (stored to x_out, default x) when
    d is given, else x. The split GEMM folds the add and the norm into its
    x pre-pass (the split GEMM's types, from 5-16 tokens by matrix size); with
    fewer tokens the fused decode GEMV takes them in its prologue.

    rope = {"n": 1 or 2, "head_dim": D, "mode": ROPE_NEOX / ROPE_INTERLEAVED,
    "pos": int32 [n_tok], "inv_freq": [D/2]} also rotates the first n outputs
    (q, k) over every channel: in the fused GEMV's epilogue when it takes
    the call, else by the RoPE pass after the projections."""
    if not 1 <= len(ws) <= 4 or len(ys) != len(ws) or len(n_rows) != len(ws):
        raise ValueError("norm_matmul: 1 to 4 matrices, with as many outputs and row counts")
    if d is not None and x_out is None:
        x_out = x
    for a, name in ((x, "x"), (d, "d"), (x_out, "x_out")):
        _need(a, n_tok * n_cols, np.float32, name)
    _need(norm_w, n_cols, np.float32, "norm_w")
    for y, nr in zip(ys, n_rows):
        _need(y, n_tok * nr, np.float32, "y")
    k = len(ws)
    wp = (ctypes.c_void_p * k)(*[w.ptr for w in ws])
    wb = (ctypes.c_int64 * k)(*[w.nbytes for w in ws])
    nr = (ctypes.c_int64 * k)(*[int(n) for n in n_rows])
    yp = (ctypes.c_void_p * k)(*[y.ptr for y in ys])
    L = _lib.lib()
    wsb = L.aero_hip_norm_matmul_workspace(int(dtype), n_cols, 0, n_tok)
    wsb += L.aero_hip_split_partials_bytes(int(sum(int(r) for r in n_rows)), n_cols, n_tok)
    buf = _norm_mm_ws.get(wsb)
    if rope is None:
        _lib.check(L.aero_hip_norm_matmul(int(dtype), k, wp, wb, nr, yp, x.ptr, as_ptr(d),
                                          as_ptr(x_out), as_ptr(norm_w), float(eps),
                                          _norm_flag(norm, unit_offset), n_cols, n_tok,
                                          as_ptr(buf), 0 if buf is None else buf.nbytes,
                                          _s(stream)), "norm_matmul")
        return
    D = int(rope["head_dim"])
    _need(rope["pos"], n_tok, np.int32, "rope pos")
    _need(rope["inv_freq"], D // 2, np.float32, "rope inv_freq")
    _lib.check(L.aero_hip_norm_matmul_rope(int(dtype), k, wp, wb, nr, yp, x.ptr, as_ptr(d),
                                           as_ptr(x_out), as_ptr(norm_w), float(eps),
                                           _norm_flag(norm, unit_offset), n_cols, n_tok,
                                           int(rope["n"]), D, int(rope.get("mode", ROPE_NEOX)),
                                           rope["pos"].ptr, rope["inv_freq"].ptr, as_ptr(buf),
                                           0 if buf is None else buf.nbytes, _s(stream)),
               "norm_matmul_rope")


def attn_input(dtype: int, ws: list, ys: list, n_rows: list, n_cols: int, n_tok: int,
               x_out: DeviceArray, x: DeviceArray | None = None, d: DeviceArray | None = None,
               emb: dict | None = None, norm_w: DeviceArray | None = None, eps: float = 1e-5,
               norm: bool = True, unit_offset: bool = False, rope: dict | None = None,
               stream: Stream | None = None) -> None:
    """The attention sublayer's input (aero_hip_attn_input): x' = the
    embedding rows (emb) or x + d (d None: x), stored to x_out; ys[m] =
    rmsnorm(x') @ W_m^T for 1-4 matrices; then the per-head norm and RoPE of
    the first rope["n"] outputs (q, k).

    emb = {"type": ggml type, "table": DeviceArray, "vocab": V, "ids": int32
    [n_tok], "scale": s (applied when > 0)}.
    rope = {"n": 1 or 2, "head_dim": D, "n_rot": rotated channels (default
    D; 0: none), "mode": ROPE_NEOX / ROPE_INTERLEAVED, "pos": int32 [n_tok],
    "inv_freq": [n_rot/2], "q_norm_w" / "k_norm_w": [D] or None, "eps",
    "unit_offset": bool}.

    With the split GEMM the embedding rows are read by its pre-pass and the
    per-head norm + RoPE run in its epilogue (heads of up to 128 rows); other
    paths run the same steps as separate passes."""
    if not 1 <= len(ws) <= 4 or len(ys) != len(ws) or len(n_rows) != len(ws):
        raise ValueError("attn_input: 1 to 4 matrices, with as many outputs and row counts")
    if emb is None and x is None:
        raise ValueError("attn_input: x or emb is needed")
    if emb is not None and d is not None:
        raise ValueError("attn_input: the embedding rows take no residual input")
    for a, name in ((x, "x"), (d, "d"), (x_out, "x_out")):
        _need(a, n_tok * n_cols, np.float32, name)
    _need(norm_w, n_cols, np.float32, "norm_w")
    for y, nr in zip(ys, n_rows):
        _need(y, n_tok * nr, np.float32, "y")
    k = len(ws)
    wp = (ctypes.c_void_p * k)(*[w.ptr for w in ws])
    wb = (ctypes.c_int64 * k)(*[w.nbytes for w in ws])
    nr = (ctypes.c_int64 * k)(*[int(n) for n in n_rows])
    yp = (ctypes.c_void_p * k)(*[y.ptr for y in ys])
    a = _lib.AttnInput()
    a.dtype, a.n_mat, a.w, a.w_bytes, a.n_rows, a.y = int(dtype), k, wp, wb, nr, yp
    a.n_cols, a.n_tok = int(n_cols), int(n_tok)
    a.x, a.d, a.x_out = as_ptr(x), as_ptr(d), x_out.ptr
    if emb is not None:
        _need(emb["ids"], n_tok, np.int32, "emb ids")
        a.emb_type, a.emb, a.emb_bytes = int(emb["type"]), emb["table"].ptr, emb["table"].nbytes
        a.vocab, a.ids = int(emb["vocab"]), emb["ids"].ptr
        a.emb_scale = float(emb.get("scale", 0.0))
    a.norm_w, a.eps, a.norm = as_ptr(norm_w), float(eps), _norm_flag(norm, unit_offset)
    if rope is not None:
        D = int(rope["head_dim"])
        n_rot = int(rope.get("n_rot", D))
        _need(rope["pos"], n_tok, np.int32, "rope pos")
        if n_rot > 0:
            _need(rope["inv_freq"], n_rot // 2, np.float32, "rope inv_freq")
        for key in ("q_norm_w", "k_norm_w"):
            _need(rope.get(key), D, np.float32, key)
        a.n_rope, a.head_dim, a.n_rot = int(rope["n"]), D, n_rot
        a.rope_mode = int(rope.get("mode", ROPE_NEOX))
        a.pos = rope["pos"].ptr
        a.inv_freq = as_ptr(rope.get("inv_freq") if n_rot > 0 else None)
        a.q_norm_w, a.k_norm_w = as_ptr(rope.get("q_norm_w")), as_ptr(rope.get("k_norm_w"))
        a.qk_eps = float(rope.get("eps", eps))
        a.qk_flags = NORM_UNIT_OFFSET if rope.get("unit_offset") else 0
    L = _lib.lib()
    wsb = L.aero_hip_norm_matmul_workspace(int(dtype), n_cols, 0, n_tok)
    wsb += L.aero_hip_split_partials_bytes(int(sum(int(r) for r in n_rows)), n_cols, n_tok)
    buf = _norm_mm_ws.get(wsb)
    _lib.check(L.aero_hip_attn_input(ctypes.byref(a), as_ptr(buf),
                                     0 if buf is None else buf.nbytes, _s(stream)),
               "attn_input")


def norm_matmul_gate_up(dtype: int, w_gate: DeviceArray, w_up: DeviceArray, x: DeviceArray,
                        out: DeviceArray, n_ff: int, n_cols: int, n_tok: int, act="silu",
                        norm_w: DeviceArray | None = None, eps: float = 1e-5,
                        norm: bool = True, unit_offset: bool = False,
                        d: DeviceArray | None = None, x_out: DeviceArray | None = None,
                        stream: Stream | None = None) -> None:
    """out = act(rmsnorm(x') @ Wg^T) * (rmsnorm(x') @ Wu^T), any token count,
    x' as norm_matmul. The split GEMM forms act(gate)*up in its epilogue."""
    kind = ACTS[act] if isinstance(act, str) else int(act)
    if w_gate.nbytes != w_up.nbytes:
        raise ValueError("norm_matmul_gate_up: gate and up must be the same size")
    if d is not None and x_out is None:
        x_out = x
    for a, name in ((x, "x"), (d, "d"), (x_out, "x_out")):
        _need(a, n_tok * n_cols, np.float32, name)
    _need(out, n_tok * n_ff, np.float32, "out")
    _need(norm_w, n_cols, np.float32, "norm_w")
    L = _lib.lib()
    wsb = L.aero_hip_norm_matmul_workspace(int(dtype), n_cols, n_ff, n_tok)
    wsb += L.aero_hip_split_partials_bytes(2 * n_ff, n_cols, n_tok)
    buf = _norm_mm_ws.get(wsb)
    _lib.check(L.aero_hip_norm_matmul_gate_up(int(dtype), w_gate.ptr, w_up.ptr, w_gate.nbytes,
                                              x.ptr, as_ptr(d), as_ptr(x_out), as_ptr(norm_w),
                                              float(eps), _norm_flag(norm, unit_offset), kind,
                                              out.ptr, n_ff, n_cols, n_tok, as_ptr(buf),
                                              0 if buf is None else buf.nbytes, _s(stream)),
               "norm_matmul_gate_up")


KV_F32, KV_INT8, KV_INT4 = 0, 1, 2


def kv_vec_bytes(dt: int, dim: int) -> int:
    """Bytes of one (position, head) vector in a KV slot of type dt."""
    return {KV_F32: 4 * dim, KV_INT8: dim, KV_INT4: dim // 2}[dt]


def kv_write(dt: int, x: DeviceArray, n_tok: int, heads: int, dim: int, q: DeviceArray,
             scale: DeviceArray | None, phys0: int, cap: int,
             stream: Stream | None = None) -> None:
    """Append rows (t, h) of x [n_tok, heads, dim] to a KV slot q [cap, heads, dim]
    (fp32 / int8 / int4, with one fp32 scale per vector in `scale` for the
    integer types) at physical positions (phys0 + t) % cap
    (include/aero/kv.hpp:62-126)."""
    if dt not in (KV_F32, KV_INT8, KV_INT4):
        raise ValueError(f"kv dtype {dt}")
    _need(x, n_tok * heads * dim, np.float32, "x")
    if q.nbytes < cap * heads * kv_vec_bytes(dt, dim):
        raise ValueError("kv slot too small")
    if dt != KV_F32:
        _need(scale, cap * heads, np.float32, "scale")
    _lib.check(_lib.lib().aero_hip_kv_write(dt, x.ptr, n_tok, heads, dim, phys0, cap, q.ptr,
                                            as_ptr(scale), _s(stream)), "kv_write")


_attn_ws = Workspace("attention chunk partials")


def attention(q: DeviceArray, k: DeviceArray, v: DeviceArray, out: DeviceArray, n_q: int,
              n_head: int, n_head_kv: int, head_dim: int, value_dim: int, n_kv: int,
              scale: float, qpos: DeviceArray | None = None, kpos: DeviceArray | None = None,
              window: int = 0, kv_dt: int = KV_F32, k_scale: DeviceArray | None = None,
              v_scale: DeviceArray | None = None, stream: Stream | None = None) -> None:
    """GQA attention with an online softmax over a KV cache
    (src/transformer.cpp:120-214): q [n_q, n_head, head_dim] -> out
    [n_q, n_head, value_dim]; K / V [n_kv, n_head_kv, dim] in kv_dt. The
    decode split's workspace is allocated once per size and reused."""
    _need(q, n_q * n_head * head_dim, np.float32, "q")
    _need(out, n_q * n_head * value_dim, np.float32, "out")
    _need(qpos, n_q, np.int32, "qpos")
    _need(kpos, n_kv, np.int32, "kpos")
    if kv_dt == KV_F32:
        _need(k, n_kv * n_head_kv * head_dim, np.float32, "k")
        _need(v, n_kv * n_head_kv * value_dim, np.float32, "v")
    else:
        if k.nbytes < n_kv * n_head_kv * kv_vec_bytes(kv_dt, head_dim) or \
                v.nbytes < n_kv * n_head_kv * kv_vec_bytes(kv_dt, value_dim):
            raise ValueError("K / V cache too small")
        _need(k_scale, n_kv * n_head_kv, np.float32, "k_scale")
        _need(v_scale, n_kv * n_head_kv, np.float32, "v_scale")
    L = _lib.lib()
    wsb = int(L.aero_hip_attention_workspace(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv))
    ws = _attn_ws.get(wsb)
    _lib.check(L.aero_hip_attention(q.ptr, kv_dt, k.ptr, as_ptr(k_scale), v.ptr,
                                    as_ptr(v_scale), out.ptr, n_q, n_head, n_head_kv, head_dim,
                                    value_dim, float(scale), as_ptr(qpos), as_ptr(kpos), n_kv,
                                    int(window), as_ptr(ws), ws.nbytes if ws is not None else 0,
                                    _s(stream)), "attention")


def softmax_rows(x: DeviceArray, y: DeviceArray, n_rows: int, n_cols: int,
                 stream: Stream | None = None) -> None:
    """y[r] = softmax(x[r]) (src/tensor.cpp:167-178); y may be x."""
    _need(x, n_rows * n_cols, np.float32, "x")
    _need(y, n_rows * n_cols, np.float32, "y")
    _lib.check(_lib.lib().aero_hip_softmax_rows(x.ptr, y.ptr, n_rows, n_cols, _s(stream)),
               "softmax_rows")


_ssm_ws = Workspace("DeltaNet scan")


def ssm_scan(q: DeviceArray, k: DeviceArray, v: DeviceArray, alpha: DeviceArray,
             beta: DeviceArray, a_log: DeviceArray, dt_bias: DeviceArray, state: DeviceArray,
             outs: DeviceArray, T: int, n_k: int, n_v: int, d: int, scale: float,
             eps: float = 1e-6, strides: tuple | None = None, q_off: int = 0, k_off: int = 0,
             v_off: int = 0, stream: Stream | None = None) -> None:
    """Gated delta-rule scan over T tokens (src/ssm.cpp:69-142): q, k
    [T, n_k, d], v / outs [T, n_v, d], alpha / beta [T, n_v], a_log / dt_bias
    [n_v], state [n_v, d, d] updated in place. strides = (q, k, v) floats
    between token rows, with q / k / v starting q_off / k_off / v_off floats
    into their arrays: slices of one packed qkv buffer, as scan_strided
    (src/ssm.cpp:128-142) reads them. The workspace (normalised q / k,
    per-token decay and gate; the chunked form's operands from 128 tokens) is
    one buffer, grown when a call needs more and reused by smaller calls, so
    calls on different streams must not overlap."""
    qs, ks, vs = strides if strides is not None else (n_k * d, n_k * d, n_v * d)
    span = lambda stride, off, w: off + (T - 1) * stride + w if T > 0 else 0
    _need(q, span(qs, q_off, n_k * d), np.float32, "q")
    _need(k, span(ks, k_off, n_k * d), np.float32, "k")
    _need(v, span(vs, v_off, n_v * d), np.float32, "v")
    _need(outs, T * n_v * d, np.float32, "outs")
    _need(alpha, T * n_v, np.float32, "alpha")
    _need(beta, T * n_v, np.float32, "beta")
    _need(a_log, n_v, np.float32, "a_log")
    _need(dt_bias, n_v, np.float32, "dt_bias")
    _need(state, n_v * d * d, np.float32, "state")
    L = _lib.lib()
    ws = _ssm_ws.get(int(L.aero_hip_ssm_workspace(T, n_k, n_v, d)))
    if strides is None and q_off == k_off == v_off == 0:
        _lib.check(L.aero_hip_ssm_scan(q.ptr, k.ptr, v.ptr, alpha.ptr, beta.ptr, a_log.ptr,
                                       dt_bias.ptr, state.ptr, T, n_k, n_v, d, float(scale),
                                       float(eps), outs.ptr, as_ptr(ws),
                                       ws.nbytes if ws is not None else 0, _s(stream)),
                   "ssm_scan")
        return
    _lib.check(L.aero_hip_ssm_scan_strided(q.ptr + 4 * q_off, qs, k.ptr + 4 * k_off, ks,
                                           v.ptr + 4 * v_off, vs, alpha.ptr, beta.ptr,
                                           a_log.ptr, dt_bias.ptr, state.ptr, T, n_k, n_v, d,
                                           float(scale), float(eps), outs.ptr, as_ptr(ws),
                                           ws.nbytes if ws is not None else 0, _s(stream)),
               "ssm_scan_strided")


def ssm_conv(x: DeviceArray, w: DeviceArray, tail: DeviceArray | None, tail_len: int,
             tail_out: DeviceArray | None, out: DeviceArray, T: int, channels: int,
             kernel: int, silu: bool = False, stream: Stream | None = None) -> int:
    """Causal depthwise conv over [tail; x] (src/ssm.cpp:173-210); the new
    history goes to tail_out (which may be tail). Returns its length. silu:
    out = silu(conv), the SSM layer's next step (src/ssm.cpp:298-301), in the
    same pass."""
    _need(x, T * channels, np.float32, "x")
    _need(out, T * channels, np.float32, "out")
    _need(w, channels * kernel, np.float32, "w")
    _need(tail, tail_len * channels, np.float32, "tail")
    _need(tail_out, (kernel - 1) * channels, np.float32, "tail_out")
    n = ctypes.c_int64()
    L = _lib.lib()
    fn = L.aero_hip_ssm_conv_silu if silu else L.aero_hip_ssm_conv
    _lib.check(fn(x.ptr, w.ptr, as_ptr(tail), int(tail_len), as_ptr(tail_out), out.ptr, T,
                  channels, kernel, ctypes.byref(n), _s(stream)),
               "ssm_conv_silu" if silu else "ssm_conv")
    return int(n.value)


def copy_f32(src: DeviceArray, dst: DeviceArray, n: int | None = None,
             stream: Stream | None = None) -> None:
    n = src.size if n is None else int(n)
    _need(src, n, np.float32, "src")
    _need(dst, n, np.float32, "dst")
    _lib.check(_lib.lib().aero_hip_copy_f32(src.ptr, dst.ptr, n, _s(stream)), "copy_f32")


def fill_f32(dst: DeviceArray, value: float, n: int | None = None,
             stream: Stream | None = None) -> None:
    """dst[:n] = value with the store-only streaming kernel."""
    n = dst.size if n is None else int(n)
    _need(dst, n, np.float32, "dst")
    _lib.check(_lib.lib().aero_hip_fill_f32(dst.ptr, float(value), n, _s(stream)), "fill_f32")
