"""GPU drop-in for the gated-DeltaNet half of the reference's
engine/native_ssm.py (libaero_ssm).

Same function names, arguments and return values as
engine/native_ssm.py:112-206 for the scan path; the arithmetic runs in
libaero_hip.so on the GPU (host arrays are staged to HBM and copied back,
synchronous):

  * softplus(x) elementwise (the scalar ABI helper, on the host);
  * delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps) with
    q/k already tiled to the value heads, returns (out, new_state) and does not
    mutate `state`;
  * scan(qh, kh, vh, ...) over T tokens, v-head h reading k-head h % n_k,
    returns (outs, new_state);
  * conv(x, w, tail, tail_len) returns (out, new_tail, new_tail_len).

SsmUnavailable when libaero_hip.so is missing or no GPU is visible. The MoE
routines and the full layer forward of the reference module are not part of
this path and raise NotImplementedError.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float

import numpy as np

from . import _lib


class SsmUnavailable(_lib.AeroHipUnavailable):
    """libaero_hip.so is not built or no GPU is visible. Callers must fall back."""


def available() -> bool:
    return _lib.available()


def unavailable_reason() -> str:
    return _lib.unavailable_reason()


def _require():
    return _lib.lib(SsmUnavailable)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _f(a):
    return a.ctypes.data_as(POINTER(c_float))


def _check(what: str) -> None:
    err = _lib.last_error()
    if err:
        raise ValueError(f"native {what} refused: {err}")


def softplus(x) -> np.ndarray:
    """log1p(exp(-|x|)) + max(x, 0) elementwise (src/ssm.cpp:22-24)."""
    lib = _require()
    xf = np.asarray(x, dtype=np.float32)
    out = np.empty_like(xf)
    of = out.reshape(-1)
    for i, v in enumerate(xf.reshape(-1)):
        of[i] = lib.aero_ssm_softplus(float(v))
    return out


def delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """One token of the gated delta rule (engine/native_ssm.py:141-159)."""
    lib = _require()
    q, k, v = _f32(q), _f32(k), _f32(v)
    alpha, beta, a_log, dt_bias = _f32(alpha), _f32(beta), _f32(a_log), _f32(dt_bias)
    n_heads, d = int(state.shape[0]), int(state.shape[1])
    if q.size != n_heads * d or k.size != n_heads * d or v.size != n_heads * d:
        raise ValueError("delta_step: q, k, v must be (n_heads, d)")
    st = _f32(state).copy()
    out = np.empty((n_heads, d), dtype=np.float32)
    lib.aero_ssm_delta_step(_f(q), _f(k), _f(v), _f(alpha), _f(beta), _f(a_log), _f(dt_bias),
                            _f(st), n_heads, d, float(scale), float(eps), _f(out))
    _check("delta_step")
    return out, st


def scan(qh, kh, vh, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """The per-head scan over T tokens (engine/native_ssm.py:162-182)."""
    lib = _require()
    qh, kh, vh = _f32(qh), _f32(kh), _f32(vh)
    alpha, beta, a_log, dt_bias = _f32(alpha), _f32(beta), _f32(a_log), _f32(dt_bias)
    T = int(qh.shape[0])
    n_k, d = int(qh.shape[1]), int(qh.shape[2])
    n_v = int(vh.shape[1])
    st = _f32(state).copy()
    if st.size != n_v * d * d:
        raise ValueError("scan: state must be (n_v, d, d)")
    outs = np.empty((T, n_v, d), dtype=np.float32)
    lib.aero_ssm_scan(_f(qh), _f(kh), _f(vh), _f(alpha), _f(beta), _f(a_log), _f(dt_bias),
                      _f(st), T, n_k, n_v, d, float(scale), float(eps), _f(outs))
    _check("scan")
    return outs, st


def conv(x, w, tail, tail_len):
    """Causal depthwise conv step (engine/native_ssm.py:185-206)."""
    lib = _require()
    x, w = _f32(x), _f32(w)
    kernel = int(w.shape[1])
    channels = int(w.shape[0])
    T = int(x.shape[0])
    keep = max(kernel - 1, 0)
    tailbuf = np.zeros((keep, channels), dtype=np.float32)
    tl = int(tail_len)
    if tl > 0:
        tailbuf[:tl] = _f32(tail)[:tl]
    out = np.empty((T, channels), dtype=np.float32)
    c_tl = ctypes.c_int(tl)
    lib.aero_ssm_conv(_f(x), _f(w), _f(tailbuf) if keep else None, ctypes.byref(c_tl), _f(out),
                      T, channels, kernel)
    _check("conv")
    return out, tailbuf, int(c_tl.value)


def forward(*args, **kwargs):
    raise NotImplementedError("the full SSM layer forward is not part of this path")


def route(*args, **kwargs):
    raise NotImplementedError("MoE routing is not part of this path")


def expert_accum(*args, **kwargs):
    raise NotImplementedError("MoE expert accumulation is not part of this path")


def ffn_block(*args, **kwargs):
    raise NotImplementedError("the MoE FFN block is not part of this path")
