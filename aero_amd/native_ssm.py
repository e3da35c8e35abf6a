"""GPU drop-in for the gated-DeltaNet half of the reference's
engine/native_ssm.py (libaero_ssm).

The scan-path functions keep the reference module's names, arguments and
results (engine/native_ssm.py:112-206); host arrays are staged to HBM, the
kernels run, the results are copied back before the call returns.

  * softplus(x): elementwise, through the library's scalar helper (host).
  * delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps): one
    token, q and k already repeated to the value heads; gives
    (out, new_state) and leaves `state` unchanged.
  * scan(qh, kh, vh, ...): T tokens, value head h reading key head h % n_k;
    gives (outs, new_state).
  * conv(x, w, tail, tail_len): gives (out, new_tail, new_tail_len).

Fallback contract. The reference's callers catch only SsmUnavailable and then
run their numpy code (engine/ssm.py:215-221, :297-304; engine/moe.py:73-77).
So every case this module does not take raises SsmUnavailable, before any
device work: no library or GPU; a head dim the GPU scan does not implement
(anything but 64, 128 and 256); and the full layer forward and the MoE
routines, which are outside this path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float

import numpy as np

from . import _lib

# head dims the GPU delta-rule scan is built for (ssm.hip)
SCAN_HEAD_DIMS = frozenset({64, 128, 256})


class SsmUnavailable(_lib.AeroHipUnavailable):
    """Raised for anything this module does not run on the GPU: no library or
    GPU, an unsupported head dim, or a routine outside the path. Callers fall
    back to their own code on it."""


def available() -> bool:
    return _lib.available()


def unavailable_reason() -> str:
    return _lib.unavailable_reason()


def _require():
    return _lib.lib(SsmUnavailable)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return a.ctypes.data_as(POINTER(c_float))


def _raise_if_set(what: str) -> None:
    msg = _lib.last_error()
    if msg:
        raise ValueError(f"GPU {what}: {msg}")


def _head_dim_supported(d: int) -> None:
    if d not in SCAN_HEAD_DIMS:
        raise SsmUnavailable(f"the GPU delta-rule scan handles head dims "
                             f"{sorted(SCAN_HEAD_DIMS)}, not {d}")


def softplus(x) -> np.ndarray:
    """Numerically safe softplus of each element (src/ssm.cpp:22-24)."""
    lib = _require()
    src = np.asarray(x, dtype=np.float32)
    out = np.empty_like(src)
    fn = lib.aero_ssm_softplus
    out.reshape(-1)[:] = [fn(float(v)) for v in src.reshape(-1)]
    return out


def delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """One token of the gated delta rule over every value head
    (engine/native_ssm.py:141-159)."""
    n_heads, d = int(state.shape[0]), int(state.shape[1])
    _head_dim_supported(d)
    lib = _require()
    qa, ka, va = _f32(q), _f32(k), _f32(v)
    if not (qa.size == ka.size == va.size == n_heads * d):
        raise ValueError(f"delta_step: q, k and v must each hold {n_heads} x {d} values")
    gates = [_f32(a) for a in (alpha, beta, a_log, dt_bias)]
    new_state = np.array(state, dtype=np.float32, order="C", copy=True)
    out = np.empty((n_heads, d), np.float32)
    lib.aero_ssm_delta_step(_fp(qa), _fp(ka), _fp(va), *[_fp(g) for g in gates],
                            _fp(new_state), n_heads, d, float(scale), float(eps), _fp(out))
    _raise_if_set("delta_step")
    return out, new_state


def scan(qh, kh, vh, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6):
    """The delta rule over T tokens, each value head with its key head
    (engine/native_ssm.py:162-182)."""
    qa, ka, va = _f32(qh), _f32(kh), _f32(vh)
    T, n_k, d = (int(s) for s in qa.shape)
    n_v = int(va.shape[1])
    _head_dim_supported(d)
    lib = _require()
    new_state = np.array(state, dtype=np.float32, order="C", copy=True)
    if new_state.size != n_v * d * d:
        raise ValueError(f"scan: the state must hold {n_v} x {d} x {d} values")
    gates = [_f32(a) for a in (alpha, beta, a_log, dt_bias)]
    outs = np.empty((T, n_v, d), np.float32)
    lib.aero_ssm_scan(_fp(qa), _fp(ka), _fp(va), *[_fp(g) for g in gates], _fp(new_state),
                      T, n_k, n_v, d, float(scale), float(eps), _fp(outs))
    _raise_if_set("scan")
    return outs, new_state


def conv(x, w, tail, tail_len):
    """Causal depthwise convolution of T new rows, continuing from the
    previous call's tail (engine/native_ssm.py:185-206)."""
    lib = _require()
    xa, wa = _f32(x), _f32(w)
    channels, width = int(wa.shape[0]), int(wa.shape[1])
    T = int(xa.shape[0])
    hist = max(width - 1, 0)
    carried = np.zeros((hist, channels), np.float32)
    n_old = int(tail_len)
    if n_old > 0:
        carried[:n_old] = _f32(tail)[:n_old]
    out = np.empty((T, channels), np.float32)
    n_tail = ctypes.c_int(n_old)
    lib.aero_ssm_conv(_fp(xa), _fp(wa), _fp(carried) if hist else None, ctypes.byref(n_tail),
                      _fp(out), T, channels, width)
    _raise_if_set("conv")
    return out, carried, int(n_tail.value)


def _outside(name: str, why: str = "use the caller's own implementation"):
    def f(*args, **kwargs):
        raise SsmUnavailable(f"native_ssm.{name} is outside the GPU path; {why}")
    f.__name__ = name
    return f


# the SSM layer runs device-resident (aero_amd.ssm_layer.SsmStep: weights, state
# and conv history kept in HBM); a host-pointer entry would upload every
# weight on each call, slower than the caller's own CPU path
forward = _outside("forward", "run the layer device-resident with aero_amd.ssm_layer.SsmStep "
                              "(weights, state and conv history in HBM)")
route = _outside("route")
expert_accum = _outside("expert_accum")
ffn_block = _outside("ffn_block")
