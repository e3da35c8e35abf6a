"""HBM buffers, streams and events over libaero_hip's runtime helpers.

No PyTorch: a DeviceArray is a hipMalloc'd buffer with a numpy-style shape and
dtype, created from or copied back to a numpy array. `ptr` is the raw device
address passed to the aero_hip_* entry points.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _lib


class DeviceArray:
    """A contiguous array in HBM. Owns its allocation unless created as a view."""

    __slots__ = ("ptr", "shape", "dtype", "nbytes", "_owner", "_base")

    def __init__(self, shape, dtype=np.float32, *, _ptr=None, _owner=True, _base=None):
        self.shape = tuple(int(d) for d in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        n = 1
        for d in self.shape:
            if d < 0:
                raise ValueError(f"negative dimension in {self.shape}")
            n *= d
        self.nbytes = n * self.dtype.itemsize
        self._base = _base
        if _ptr is not None:
            self.ptr = _ptr
            self._owner = _owner
            return
        L = _lib.lib()
        p = L.aero_hip_malloc(max(self.nbytes, 256))
        if not p:
            raise MemoryError(f"hipMalloc of {self.nbytes} bytes failed: {_lib.last_error()}")
        self.ptr = p
        self._owner = True

    # ------------------------------------------------------------ creation
    @classmethod
    def empty(cls, shape, dtype=np.float32) -> "DeviceArray":
        return cls(shape, dtype)

    @classmethod
    def from_numpy(cls, a) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.copy_from(a)
        return d

    def view(self, shape=None, dtype=None, offset_bytes: int = 0) -> "DeviceArray":
        """A non-owning view at `offset_bytes` into this buffer."""
        shape = self.shape if shape is None else shape
        dtype = self.dtype if dtype is None else dtype
        v = DeviceArray(shape, dtype, _ptr=self.ptr + offset_bytes, _owner=False, _base=self)
        if offset_bytes < 0 or offset_bytes + v.nbytes > self.nbytes:
            raise ValueError("view outside the parent buffer")
        return v

    # ------------------------------------------------------------ transfer
    def copy_from(self, a) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: host {a.nbytes} B vs device {self.nbytes} B")
        _lib.check(_lib.lib().aero_hip_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes),
                   "memcpy H2D")

    def clone(self) -> "DeviceArray":
        """A new allocation holding a device-to-device copy of this one
        (complete when this returns)."""
        d = DeviceArray(self.shape, self.dtype)
        L = _lib.lib()
        _lib.check(L.aero_hip_memcpy_dtod(d.ptr, self.ptr, self.nbytes, None), "memcpy D2D")
        _lib.check(L.aero_hip_stream_synchronize(None), "stream synchronize")
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.check(_lib.lib().aero_hip_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes),
                   "memcpy D2H")
        return out

    @property
    def size(self) -> int:
        return self.nbytes // self.dtype.itemsize

    def free(self) -> None:
        if self._owner and self.ptr:
            L = _lib.load()
            if L is not None:
                L.aero_hip_free(self.ptr)
        self.ptr = 0
        self._owner = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self.ptr or 0:x})"


def as_ptr(x):
    """Device address of a DeviceArray, None for None; ints pass through."""
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    if isinstance(x, int):
        return x
    raise TypeError(f"expected a DeviceArray, got {type(x).__name__}")


class Stream:
    """A HIP stream at default priority (NULL handle = the null stream)."""

    def __init__(self, null: bool = False):
        self.handle = None if null else _lib.lib().aero_hip_stream_create()
        if not null and not self.handle:
            raise _lib.AeroHipError(f"stream create: {_lib.last_error()}")

    def synchronize(self) -> None:
        _lib.check(_lib.lib().aero_hip_stream_synchronize(self.handle), "stream sync")

    def destroy(self) -> None:
        if self.handle:
            _lib.lib().aero_hip_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        self.handle = _lib.lib().aero_hip_event_create()
        if not self.handle:
            raise _lib.AeroHipError(f"event create: {_lib.last_error()}")

    def record(self, stream: Stream | None = None) -> None:
        _lib.check(_lib.lib().aero_hip_event_record(self.handle, stream.handle if stream else None),
                   "event record")

    def synchronize(self) -> None:
        _lib.check(_lib.lib().aero_hip_event_synchronize(self.handle), "event sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = _lib.lib().aero_hip_event_elapsed_ms(self.handle, end.handle)
        if ms < 0:
            raise _lib.AeroHipError(f"event elapsed: {_lib.last_error()}")
        return float(ms)

    def destroy(self) -> None:
        if self.handle:
            _lib.lib().aero_hip_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Plan:
    """A recorded sequence of aero_hip_* device ops, replayed with one call.

        plan = Plan()
        with plan:                       # ops are checked and recorded, not run
            ops.rmsnorm(x, w, h, R, N, eps)
            ops.act_mul("silu", g, u, o)
        plan.launch(stream)              # issues the recorded kernels in order

    The caller's buffers an op was recorded with must outlive the plan: the
    caller holds them. Library-owned scratch buffers (Workspace) that ops use
    while the plan records are held by the plan itself, so a later, larger
    call that replaces such a buffer cannot free memory the plan still
    writes.
    """

    def __init__(self):
        self.handle = _lib.lib().aero_hip_plan_create()
        if not self.handle:
            raise MemoryError("plan create failed")
        self._held: list = []

    def __enter__(self):
        _lib.check(_lib.lib().aero_hip_plan_begin(self.handle), "plan_begin")
        _recording.plan = self
        return self

    def __exit__(self, *exc):
        _recording.plan = None
        _lib.check(_lib.lib().aero_hip_plan_end(self.handle), "plan_end")
        return False

    def hold(self, buf) -> None:
        """Keep `buf` alive as long as this plan exists."""
        if not any(b is buf for b in self._held):
            self._held.append(buf)

    def __len__(self) -> int:
        return int(_lib.lib().aero_hip_plan_size(self.handle))

    def event_arrays(self, starts, stops):
        """ctypes arrays of event handles for launch(), one pair per kernel."""
        n = len(self)
        if len(starts) != n or len(stops) != n:
            raise ValueError(f"need {n} start and stop events")
        arr = ctypes.c_void_p * n
        return arr(*[e.handle for e in starts]), arr(*[e.handle for e in stops])

    def launch(self, stream: "Stream | None" = None, events=None) -> None:
        a, b = (None, None) if events is None else events
        _lib.check(_lib.lib().aero_hip_plan_launch(self.handle, stream.handle if stream else None,
                                                   a, b), "plan_launch")

    def destroy(self) -> None:
        if self.handle:
            L = _lib.load()
            if L is not None:
                L.aero_hip_plan_destroy(self.handle)
            self.handle = None
        self._held = []

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


_recording = threading.local()


def recording_plan() -> "Plan | None":
    """The plan this thread is recording into, if any."""
    return getattr(_recording, "plan", None)


class Workspace:
    """Device scratch memory for one family of ops (split GEMM, attention,
    DeltaNet scan): one buffer, grown to the largest request seen and never
    shrunk, so alternating sizes (a prefill layer's 4096- and 14336-column
    GEMMs) reuse it instead of freeing and reallocating (hipFree waits for
    the device). A buffer used while a plan records is held by that plan.
    Calls that share a workspace must not run concurrently on different
    streams: they would share its contents."""

    def __init__(self, what: str):
        self.what = what
        self.buf: DeviceArray | None = None

    def get(self, nbytes: int) -> "DeviceArray | None":
        if nbytes <= 0:
            return None
        if self.buf is None or self.buf.nbytes < nbytes:
            self.buf = None                    # drop ours before allocating the larger one
            self.buf = DeviceArray.empty(-(-int(nbytes) // 4), np.float32)
        plan = recording_plan()
        if plan is not None:
            plan.hold(self.buf)
        return self.buf


def time_next_kernel(start: Event, stop: Event) -> None:
    """The next kernel launched by an aero_hip_* op on this thread records its
    own device begin/end timestamps into start/stop."""
    _lib.check(_lib.lib().aero_hip_time_next_kernel(start.handle, stop.handle), "time_next_kernel")


def synchronize() -> None:
    _lib.check(_lib.lib().aero_hip_device_synchronize(), "device sync")


def device_count() -> int:
    L = _lib.load()
    return 0 if L is None else int(L.aero_hip_device_count())


def tune_set(key: str, value: int | None) -> None:
    """Override one launch-shape knob for the rest of the process (None drops
    the override, so the built-in default applies). Plans keep the kernel
    choice they recorded."""
    _lib.check(_lib.lib().aero_hip_tune_set(key.encode(), 0 if value is None else int(value),
                                            1 if value is None else 0), "tune_set")
