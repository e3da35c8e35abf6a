"""GPU drop-in for the reference's engine/native.py (libaero_kernels): whole-
tensor dequantisation and the quantised matvec / matmul.

Kept from engine/native.py:22-285 as its contract: the DTYPE_* constants,
NATIVE_TYPES (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS: :33-34), KernelsUnavailable,
available(), unavailable_reason(), block_bytes(), block_values(),
hardware_threads(), hw_threads(), dequant(dtype, raw, shape, threads=0),
matvec(dtype, w_bytes, x) and matmul(dtype, w_bytes, X).

Quantised input may be bytes, bytearray, memoryview or a uint8 ndarray. A
type outside NATIVE_TYPES, or fewer bytes than the requested values need,
raises ValueError before anything reaches the GPU. The weight is uploaded on
every matvec / matmul call, since the reference's signature carries no
device handle; a model loop keeps weights resident and calls
aero_amd.ops.matvec instead.
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

NATIVE_TYPES = frozenset({DTYPE_Q8_0, DTYPE_Q4_K, DTYPE_Q5_K, DTYPE_Q6_K, DTYPE_IQ4_XS})

# (values, bytes) per block of each GGML type this module knows
_GEOMETRY = {DTYPE_F32: (1, 4), DTYPE_F16: (1, 2), DTYPE_BF16: (1, 2), DTYPE_Q8_0: (32, 34),
             DTYPE_Q4_K: (256, 144), DTYPE_Q5_K: (256, 176), DTYPE_Q6_K: (256, 210),
             DTYPE_IQ4_XS: (256, 136)}


class KernelsUnavailable(_lib.AeroHipUnavailable):
    """Raised when libaero_hip.so cannot be used (not built, or no GPU)."""


def available() -> bool:
    return _lib.available()


def unavailable_reason() -> str:
    return _lib.unavailable_reason()


def _require():
    return _lib.lib(KernelsUnavailable)


def _loaded():
    L = _lib.load()
    if L is None:
        raise KernelsUnavailable(_lib.unavailable_reason())
    return L


def block_bytes(dtype: int) -> int:
    """Bytes of one block of `dtype` (0 for a type the library does not know)."""
    return int(_loaded().aero_dtype_block_bytes(int(dtype)))


def block_values(dtype: int) -> int:
    """Values held by one block of `dtype` (0 for an unknown type)."""
    return int(_loaded().aero_dtype_block_values(int(dtype)))


def hardware_threads() -> int:
    L = _lib.load()
    return 1 if L is None else int(L.aero_hardware_threads())


_cached_threads = 0


def hw_threads() -> int:
    """The reference's auto thread count (min(cores, 8)), looked up once; 0
    without the library. The GPU path does not use it."""
    global _cached_threads
    if not _cached_threads:
        L = _lib.load()
        if L is None:
            return 0
        _cached_threads = int(L.aero_hardware_threads())
    return _cached_threads


def _byte_view(raw):
    """(pointer, owner) for quantised input; `owner` keeps a temporary alive
    for the duration of the call. bytes are immutable, so they are copied."""
    if isinstance(raw, np.ndarray):
        if raw.dtype != np.uint8:
            raise TypeError(f"quantised input must be uint8, not {raw.dtype}")
        flat = np.ascontiguousarray(raw).reshape(-1)
        return flat.ctypes.data_as(POINTER(c_uint8)), flat
    if isinstance(raw, bytes):
        buf = (c_uint8 * len(raw)).from_buffer_copy(raw)
        return buf, buf
    if isinstance(raw, (bytearray, memoryview)):
        buf = (c_uint8 * len(raw)).from_buffer(raw)
        return buf, buf
    raise TypeError(f"quantised input must be bytes-like, not {type(raw).__name__}")


def _byte_len(raw) -> int:
    return int(raw.nbytes) if isinstance(raw, np.ndarray) else len(raw)


def _native_type(dtype: int) -> int:
    if dtype not in NATIVE_TYPES:
        raise ValueError(f"dequant/matvec: GGML type {dtype} is not one of "
                         f"{sorted(NATIVE_TYPES)}")
    return int(dtype)


def _rows_in(w_bytes, dtype: int, n_cols: int) -> int:
    if n_cols <= 0:
        return 0
    bv, bb = _GEOMETRY[dtype]
    return (_byte_len(w_bytes) // bb) * bv // n_cols


def dequant(dtype: int, raw, shape, threads: int = 0):
    """All values of a quantised tensor as a float32 array of `shape`, computed
    on the GPU. `threads` exists for the reference's signature and is
    ignored."""
    L = _require()
    t = _native_type(dtype)
    dims = (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(int(d) for d in shape)
    n = int(np.prod(dims, dtype=np.int64)) if dims else 1
    out = np.zeros(n, np.float32)
    ptr, owner = _byte_view(raw)
    have = _byte_len(raw)
    ok = L.aero_dequant_ref(c_int(t), ptr, c_int64(have), out.ctypes.data_as(POINTER(c_float)),
                            c_int64(n))
    del owner
    if not ok:
        raise ValueError(f"dequant: the library declined type {t}, {n} values from {have} "
                         f"bytes ({_lib.last_error()})")
    return out.reshape(dims)


def matvec(dtype: int, w_bytes, x, threads: int = 1):
    """W @ x for a quantised W with x.size columns (engine/native.py:232-255);
    the row count follows from the bytes given. `threads` is ignored."""
    L = _require()
    t = _native_type(dtype)
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n_rows = _rows_in(w_bytes, t, xv.size)
    y = np.zeros(n_rows, np.float32)
    ptr, owner = _byte_view(w_bytes)
    ok = L.aero_matvec(t, ptr, xv.ctypes.data_as(POINTER(c_float)),
                       y.ctypes.data_as(POINTER(c_float)), c_int64(n_rows), c_int64(xv.size),
                       c_int(threads))
    del owner
    if not ok:
        raise ValueError(f"matvec: the library declined type {t}, {n_rows} x {xv.size} "
                         f"({_lib.last_error()})")
    return y


def matmul(dtype: int, w_bytes, X, threads: int = 1):
    """X @ W^T for a quantised W (engine/native.py:258-285): X of shape
    (T, n_cols) gives (T, n_rows)."""
    L = _require()
    t = _native_type(dtype)
    Xv = np.ascontiguousarray(X, dtype=np.float32)
    Xv = Xv.reshape(1, -1) if Xv.ndim == 1 else Xv
    T, n_cols = Xv.shape
    n_rows = _rows_in(w_bytes, t, n_cols)
    Y = np.zeros((T, n_rows), np.float32)
    ptr, owner = _byte_view(w_bytes)
    ok = L.aero_matmul(t, ptr, Xv.ctypes.data_as(POINTER(c_float)),
                       Y.ctypes.data_as(POINTER(c_float)), c_int64(T), c_int64(n_rows),
                       c_int64(n_cols), c_int(threads))
    del owner
    if not ok:
        raise ValueError(f"matmul: the library declined type {t}, {T} tokens x {n_rows} x "
                         f"{n_cols} ({_lib.last_error()})")
    return Y
