"""GPU drop-in for the reference's engine/native.py (libaero_kernels):
dequant and the quantised matvec / matmul.

Same constants, names, arguments and exceptions as engine/native.py:22-285:
DTYPE_*, NATIVE_TYPES, KernelsUnavailable, available(), unavailable_reason(),
block_bytes(), block_values(), hardware_threads(), hw_threads(), _u8(),
_raw_nbytes(), dequant(dtype, raw, shape, threads=0) -> a new float32 array
of `shape`, matvec(dtype, w_bytes, x) -> W @ x and matmul(dtype, w_bytes, X)
-> X @ W^T. raw / w_bytes may be bytes, bytearray or memoryview (or a uint8
ndarray); a short buffer or an unsupported type raises ValueError before any
device work. The host forms upload their inputs per call; a loop that keeps
weights in HBM uses aero_amd.ops.matvec.

NATIVE_TYPES is the reference's set (engine/native.py:33-34): Q8_0, Q4_K,
Q5_K, Q6_K, IQ4_XS, all dequantised on the GPU.
"""
from __future__ import annotations

from ctypes import POINTER, c_float, c_int, c_int64, c_uint8

import numpy as np

from . import _lib

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_Q8_0 = 8
DTYPE_Q4_K = 12
DTYPE_Q5_K = 13
DTYPE_Q6_K = 14
DTYPE_IQ4_XS = 23
DTYPE_BF16 = 30

NATIVE_TYPES = frozenset({DTYPE_Q8_0, DTYPE_Q4_K, DTYPE_Q5_K, DTYPE_Q6_K,
                          DTYPE_IQ4_XS})

_BLOCK_VALUES = {DTYPE_F32: 1, DTYPE_F16: 1, DTYPE_Q8_0: 32, DTYPE_Q4_K: 256,
                 DTYPE_Q5_K: 256, DTYPE_Q6_K: 256, DTYPE_IQ4_XS: 256, DTYPE_BF16: 1}
_BLOCK_BYTES = {DTYPE_F32: 4, DTYPE_F16: 2, DTYPE_Q8_0: 34, DTYPE_Q4_K: 144,
                DTYPE_Q5_K: 176, DTYPE_Q6_K: 210, DTYPE_IQ4_XS: 136, DTYPE_BF16: 2}


class KernelsUnavailable(_lib.AeroHipUnavailable):
    """libaero_hip.so is not built or no GPU is visible. Callers must fall back."""


def available() -> bool:
    return _lib.available()


def unavailable_reason() -> str:
    return _lib.unavailable_reason()


def _require():
    return _lib.lib(KernelsUnavailable)


def block_bytes(dtype: int) -> int:
    L = _lib.load()
    if L is None:
        raise KernelsUnavailable(_lib.unavailable_reason())
    return int(L.aero_dtype_block_bytes(int(dtype)))


def block_values(dtype: int) -> int:
    L = _lib.load()
    if L is None:
        raise KernelsUnavailable(_lib.unavailable_reason())
    return int(L.aero_dtype_block_values(int(dtype)))


def hardware_threads() -> int:
    L = _lib.load()
    return 1 if L is None else int(L.aero_hardware_threads())


_threads_hint = 0


def hw_threads() -> int:
    """Host thread count, cached (kept for the reference's auto-thread rule). 0
    when the library is absent."""
    global _threads_hint
    if _threads_hint:
        return _threads_hint
    L = _lib.load()
    if L is None:
        return 0
    _threads_hint = int(L.aero_hardware_threads())
    return _threads_hint


def _u8(arr):
    """uint8 ctypes view of a bytes-like object (bytes are copied)."""
    if isinstance(arr, (bytes, bytearray, memoryview)):
        if isinstance(arr, bytes):
            return (c_uint8 * len(arr)).from_buffer_copy(arr)
        return (c_uint8 * len(arr)).from_buffer(arr)
    if isinstance(arr, np.ndarray) and arr.dtype == np.uint8:
        a = np.ascontiguousarray(arr).reshape(-1)
        return a.ctypes.data_as(POINTER(c_uint8)), a
    raise TypeError(f"expected bytes-like, got {type(arr).__name__}")


def _raw_len(raw) -> int:
    """len() of the weight buffer, as the reference sizes it (bytes)."""
    return int(raw.nbytes) if isinstance(raw, np.ndarray) else len(raw)


def _raw_nbytes(raw, dtype: int, n_values: int) -> int:
    """Bytes the caller actually passed (never more)."""
    if isinstance(raw, np.ndarray):
        return int(raw.nbytes)
    try:
        return len(raw)
    except TypeError:
        pass
    bv = _BLOCK_VALUES.get(dtype, 0)
    if not bv:
        return 0
    return (n_values // bv) * _BLOCK_BYTES.get(dtype, 0)


def dequant(dtype: int, raw, shape, threads: int = 0):
    """Dequantise a whole tensor on the GPU; returns a float32 array of `shape`.

    `threads` is accepted for signature compatibility and ignored.
    """
    lib = _require()
    if dtype not in NATIVE_TYPES:
        raise ValueError(f"dtype {dtype} has no native dequantiser")
    if isinstance(shape, (int, np.integer)):
        shape = (int(shape),)
    n = 1
    for d in shape:
        n *= int(d)
    out = np.zeros(n, dtype=np.float32)
    buf = _u8(raw)
    keep = None
    if isinstance(buf, tuple):
        buf, keep = buf
    rl = c_int64(_raw_nbytes(raw, dtype, n))
    ok = lib.aero_dequant_ref(c_int(int(dtype)), buf, rl,
                              out.ctypes.data_as(POINTER(c_float)), c_int64(n))
    del keep
    if not ok:
        raise ValueError(
            f"native dequant refused dtype={dtype} n={n} raw_len={int(rl.value)} "
            f"(buffer too short, or the type/dimension combination is unsupported): "
            f"{_lib.last_error()}")
    return out.reshape(shape)


def matvec(dtype: int, w_bytes, x, threads: int = 1):
    """y = W @ x (engine/native.py:232-255). `w_bytes` is the raw quantised
    tensor, `x` a float32 array; n_rows = values in w_bytes // x.size. W is
    uploaded per call (the reference's signature holds no device handle);
    `threads` is ignored."""
    lib = _require()
    if dtype not in NATIVE_TYPES:
        raise ValueError(f"dtype {dtype} has no native kernel")
    wb = _u8(w_bytes)
    keep = None
    if isinstance(wb, tuple):
        wb, keep = wb
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n_cols = xv.size
    bv = block_values(dtype)
    n_rows = (_raw_len(w_bytes) // block_bytes(dtype)) * bv // n_cols if n_cols else 0
    y = np.zeros(n_rows, dtype=np.float32)
    ok = lib.aero_matvec(int(dtype), wb, xv.ctypes.data_as(POINTER(c_float)),
                         y.ctypes.data_as(POINTER(c_float)), c_int64(n_rows), c_int64(n_cols),
                         c_int(threads))
    del keep
    if not ok:
        raise ValueError(
            f"native matvec refused dtype={dtype} n_rows={n_rows} n_cols={n_cols}: "
            f"{_lib.last_error()}")
    return y


def matmul(dtype: int, w_bytes, X, threads: int = 1):
    """Y = X @ W^T (engine/native.py:258-285): X (T, n_cols) -> Y (T, n_rows)."""
    lib = _require()
    if dtype not in NATIVE_TYPES:
        raise ValueError(f"dtype {dtype} has no native kernel")
    wb = _u8(w_bytes)
    keep = None
    if isinstance(wb, tuple):
        wb, keep = wb
    Xv = np.ascontiguousarray(X, dtype=np.float32)
    if Xv.ndim == 1:
        Xv = Xv[None, :]
    T, n_cols = Xv.shape
    bv = block_values(dtype)
    n_rows = (_raw_len(w_bytes) // block_bytes(dtype)) * bv // n_cols if n_cols else 0
    Y = np.zeros((T, n_rows), dtype=np.float32)
    ok = lib.aero_matmul(int(dtype), wb, Xv.ctypes.data_as(POINTER(c_float)),
                         Y.ctypes.data_as(POINTER(c_float)), c_int64(T), c_int64(n_rows),
                         c_int64(n_cols), c_int(threads))
    del keep
    if not ok:
        raise ValueError(
            f"native matmul refused dtype={dtype} T={T} n_rows={n_rows} n_cols={n_cols}: "
            f"{_lib.last_error()}")
    return Y
