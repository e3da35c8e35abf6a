"""GGUF files on MI355X: the reference's reader interface (engine/gguf.py,
GGUFReader) over the library's native parser (aero_gguf_*), with tensors
uploaded to HBM and dequantised there.

    r = GGUFReader("model.gguf")
    r.kv, r.tensors, r.arch(), r.hp("block_count")          # as the reference
    w = r.tensor("blk.0.attn_norm.weight")                   # host fp32 array
    rows = r.tensor_rows(r.tensors["token_embd.weight"], 0, 8)
    emb = r.to_device("token_embd.weight")                   # resident in HBM
    emb.gather(ids, out)                                     # device row gather

Parsing (header, metadata, tensor index) runs in C++ on a read-only mapping of
the file; `to_device` reads a tensor with pread into pinned buffers and copies
it to HBM; `tensor`, `tensor_rows`, `matvec` and `matmul` compute on the GPU and
return host arrays as the reference does. There is no CPU fallback: without
the library or a GPU, construction (or the first device use) raises
`GGUFUnavailable`.
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass
from typing import Any, Dict, Tuple

import numpy as np

from . import _lib, ops
from .device import DeviceArray, Stream

MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# ggml value types (engine/gguf.py:35-38)
GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16 = 0, 1, 2, 3
GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL = 4, 5, 6, 7
GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = 8, 9, 10, 11, 12

# ggml tensor types (engine/gguf.py:41-47)
T_F32, T_F16 = 0, 1
T_Q4_0, T_Q4_1 = 2, 3
T_Q5_0, T_Q5_1 = 6, 7
T_Q8_0 = 8
T_Q4_K, T_Q5_K, T_Q6_K = 12, 13, 14
T_IQ4_XS = 23
T_BF16 = 30

TYPE_NAMES: Dict[int, str] = {
    T_F32: "F32", T_F16: "F16", T_Q4_0: "Q4_0", T_Q4_1: "Q4_1",
    T_Q5_0: "Q5_0", T_Q5_1: "Q5_1", T_Q8_0: "Q8_0",
    T_Q4_K: "Q4_K", T_Q5_K: "Q5_K", T_Q6_K: "Q6_K", T_IQ4_XS: "IQ4_XS",
    T_BF16: "BF16",
}

# types the GPU dequantises (aero_hip_dequant / aero_hip_tensor_rows), and
# those with a quantised GPU matvec (aero_hip_matvec)
DEVICE_TYPES = frozenset({T_F32, T_F16, T_BF16, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_IQ4_XS})
MATVEC_TYPES = frozenset({T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_IQ4_XS})


class GGUFUnavailable(_lib.AeroHipUnavailable):
    pass


@dataclass
class TensorInfo:
    """Where one tensor lives in the file and what it holds. `dims` are the
    extents exactly as the file lists them, innermost first; `shape` turns
    them round into numpy's outermost-first order. `offset` counts from the
    start of the data section; `nbytes` is -1 for a GGML type whose block
    geometry the library does not know. Field and property names are the
    reference reader's interface (engine/gguf.py:59-78)."""
    name: str
    dims: Tuple[int, ...]
    type_id: int
    offset: int
    n_elements: int = 0
    nbytes: int = -1

    @property
    def shape(self) -> Tuple[int, ...]:
        return self.dims[::-1]

    @property
    def type_name(self) -> str:
        known = TYPE_NAMES.get(self.type_id)
        return known if known is not None else f"ggml_type_{self.type_id}"


def _text(s: str) -> str:
    # strings arrive with each byte >= 0x80 as one code point; decode the bytes
    # as UTF-8 with replacement, as the reference reader does
    return s.encode("latin-1").decode("utf-8", "replace") if not s.isascii() else s


def _decode(v: Any) -> Any:
    if isinstance(v, str):
        return _text(v)
    if isinstance(v, list):
        return [_decode(x) for x in v]
    return v


def _require():
    L = _lib.load()
    if L is None:
        raise GGUFUnavailable(_lib.unavailable_reason())
    return L


class DeviceTensor:
    """A tensor's file bytes resident in HBM, with its row geometry."""

    def __init__(self, info: TensorInfo, raw: DeviceArray):
        self.info = info
        self.raw = raw
        self.type_id = info.type_id
        self.n_rows = GGUFReader.row_shape(info)[0]
        self.n_per_row = GGUFReader.n_row_elements(info)
        self.row_bytes = info.nbytes // max(self.n_rows, 1)

    def rows(self, r0: int, r1: int, out: DeviceArray | None = None,
             stream: Stream | None = None) -> DeviceArray:
        """fp32 rows [r0, r1) (device), engine/gguf.py:297-314 on HBM."""
        if not (0 <= r0 <= r1 <= self.n_rows):
            raise ValueError(f"row range [{r0},{r1}) outside [0,{self.n_rows})")
        if out is None:
            out = DeviceArray.empty((r1 - r0, self.n_per_row))
        elif out.dtype != np.float32 or out.size < (r1 - r0) * self.n_per_row:
            raise ValueError("out: too small or not float32")
        _lib.check(_require().aero_hip_tensor_rows(
            self.type_id, self.raw.ptr, self.raw.nbytes, self.n_rows, self.n_per_row, r0, r1,
            out.ptr, stream.handle if stream else None), "tensor_rows")
        return out

    def gather(self, ids: DeviceArray, out: DeviceArray, scale: float = 0.0,
               bad_count: DeviceArray | None = None, stream: Stream | None = None) -> None:
        """out[i] = row ids[i] (* scale): the embedding gather over this table."""
        ops.embed_gather(self.type_id, self.raw, self.n_rows, self.n_per_row, ids, out,
                         scale=scale, bad_count=bad_count, stream=stream)

    def matvec(self, x: DeviceArray, y: DeviceArray, n_tok: int = 1,
               stream: Stream | None = None) -> None:
        """y[t] = W x[t] for a resident weight (rows = outputs)."""
        ops.matvec(self.type_id, self.raw, x, y, self.n_rows, self.n_per_row, n_tok,
                   stream=stream)


class GGUFReader:
    """Random-access reader over a .gguf file (engine/gguf.py:105-445)."""

    # tensor() keeps the host result of any tensor up to this size, as the
    # reference reader does for norms and biases (engine/gguf.py:274-275)
    SMALL_TENSOR_BYTES = 1 << 20

    def __init__(self, path: str) -> None:
        L = _require()
        self.path = path
        self._h = L.aero_gguf_open(path.encode())
        if not self._h:
            msg = _lib.last_error()
            if "cannot open" in msg:
                raise FileNotFoundError(msg)
            raise ValueError(msg)
        self.version = int(L.aero_gguf_version(self._h))
        self.alignment = int(L.aero_gguf_alignment(self._h))
        self.data_offset = int(L.aero_gguf_data_offset(self._h))
        n = ctypes.c_int64()
        p = L.aero_gguf_kv_json(self._h, ctypes.byref(n))
        entries = json.loads(ctypes.string_at(p, n.value).decode("ascii"))
        self.kv: Dict[str, Any] = {}
        self.kv_types: Dict[str, int] = {}
        for key, vtype, value in entries:
            k = _text(key)
            self.kv[k] = _decode(value)
            self.kv_types[k] = int(vtype)
        self.tensors: Dict[str, TensorInfo] = {}
        self._cnames: Dict[str, bytes] = {}   # name as the file's bytes
        t_type, t_nd = ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_int64 * 4)()
        off, nb = ctypes.c_int64(), ctypes.c_int64()
        for i in range(int(L.aero_gguf_n_tensors(self._h))):
            name_b = ctypes.string_at(L.aero_gguf_tensor_name(self._h, i))
            L.aero_gguf_tensor_info(self._h, name_b, ctypes.byref(t_type), ctypes.byref(t_nd),
                                    dims, ctypes.byref(off), ctypes.byref(nb))
            d = tuple(int(dims[j]) for j in range(t_nd.value))
            n_el = 1
            for x in d:
                n_el *= x
            name = _text(name_b.decode("latin-1"))
            if name not in self.tensors:
                self.tensors[name] = TensorInfo(name, d, int(t_type.value), int(off.value),
                                                n_el, int(nb.value))
                self._cnames[name] = name_b
        self._small_cache: Dict[str, np.ndarray] = {}
        self._small_bytes = 0
        self._resident: Dict[str, DeviceTensor] = {}

    # ---- lifetime --------------------------------------------------------
    def summary(self) -> str:
        """A short human-readable description: the file, its format version,
        architecture and counts, then every scalar hyperparameter stored under
        the architecture's prefix, sorted by name."""
        arch = self.arch()
        head = (f"{self.path}: GGUF v{self.version}, architecture '{arch}', "
                f"{len(self.tensors)} tensors, {len(self.kv)} metadata entries")
        prefix = arch + "."
        body = [f"  {k[len(prefix):]} = {v}" for k, v in sorted(self.kv.items())
                if k.startswith(prefix) and isinstance(v, (int, float, str, bool))]
        return "\n".join([head] + body)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._resident.clear()
            L = _lib.load()
            if L is not None:
                L.aero_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- metadata (engine/gguf.py:221-230 is the interface) ---------------
    def get(self, key: str, default: Any = None) -> Any:
        """The value stored under the full key `key`, else `default`."""
        return self.kv.get(key, default)

    def arch(self) -> str:
        """general.architecture, or "unknown" when the file has none."""
        return str(self.kv.get("general.architecture", "unknown"))

    def hp(self, suffix: str, default: Any = None) -> Any:
        """The value under "<architecture>.<suffix>" (for a llama file,
        hp("context_length") reads llama.context_length), else `default`."""
        return self.kv.get(self.arch() + "." + suffix, default)

    # ---- tensor access -----------------------------------------------------
    def _cname(self, info: TensorInfo) -> bytes:
        return self._cnames[info.name]

    def _known(self, info: TensorInfo) -> None:
        if info.nbytes < 0:
            raise NotImplementedError(f"unsupported ggml type {info.type_id}")

    def tensor_bytes(self, info: TensorInfo) -> bytes:
        """Raw bytes of one tensor (engine/gguf.py:232-237)."""
        self._known(info)
        buf = ctypes.create_string_buffer(max(info.nbytes, 1))
        _lib.check(_require().aero_gguf_read(self._h, self._cname(info), 0, info.nbytes, buf),
                   "gguf read")
        return buf.raw[:info.nbytes]

    def to_device(self, name: str, stream: Stream | None = None) -> DeviceTensor:
        """Upload a tensor's bytes to HBM once; later calls return the same
        resident copy."""
        dt = self._resident.get(name)
        if dt is not None:
            return dt
        info = self.tensors[name]
        self._known(info)
        raw = DeviceArray.empty(max(info.nbytes, 1), np.uint8)
        _lib.check(_require().aero_gguf_upload(self._h, self._cname(info), 0, info.nbytes,
                                               raw.ptr, stream.handle if stream else None),
                   "gguf upload")
        dt = self._resident[name] = DeviceTensor(info, raw)
        return dt

    def release(self, name: str) -> None:
        """Drop a resident copy made by to_device."""
        self._resident.pop(name, None)

    def _device_type(self, info: TensorInfo) -> None:
        self._known(info)
        if info.type_id not in DEVICE_TYPES:
            raise NotImplementedError(f"no GPU dequantiser for {info.type_name}")

    def tensor(self, name: str) -> np.ndarray:
        """One tensor dequantised on the GPU to a float32 array of its
        row-major shape (engine/gguf.py:239-272); small tensors are memoised."""
        hit = self._small_cache.get(name)
        if hit is not None:
            return hit
        info = self.tensors[name]
        self._device_type(info)
        dt = self._resident.get(name)
        raw = dt.raw if dt is not None else self._upload_range(info, 0, info.nbytes)
        out = DeviceArray.empty(max(info.n_elements, 1))
        ops.dequant(info.type_id, raw, out, info.n_elements)
        res = out.numpy()[:info.n_elements].reshape(info.shape)
        if res.nbytes <= self.SMALL_TENSOR_BYTES:
            self._small_cache[name] = res
            self._small_bytes += res.nbytes
        return res

    @property
    def small_cache_bytes(self) -> int:
        return self._small_bytes

    def _upload_range(self, info: TensorInfo, b0: int, nbytes: int) -> DeviceArray:
        raw = DeviceArray.empty(max(nbytes, 1), np.uint8)
        _lib.check(_require().aero_gguf_upload(self._h, self._cname(info), b0, nbytes, raw.ptr,
                                               None), "gguf upload")
        return raw

    def row_bytes(self, info: TensorInfo) -> int:
        """Bytes per row (engine/gguf.py:278-283)."""
        self._known(info)
        n_rows, _ = self.row_shape(info)
        return info.nbytes // max(n_rows, 1)

    @staticmethod
    def n_row_elements(info: TensorInfo) -> int:
        n_rows, _ = GGUFReader.row_shape(info)
        return info.n_elements // n_rows

    @staticmethod
    def row_shape(info: TensorInfo) -> Tuple[int, int]:
        """(n_rows, n_per_row). A 1-D tensor is one row (engine/gguf.py:290-295)."""
        if len(info.shape) <= 1:
            return 1, int(info.shape[0]) if info.shape else 0
        return int(info.shape[0]), int(info.shape[1])

    def tensor_rows(self, info: TensorInfo, r0: int, r1: int) -> np.ndarray:
        """Rows [r0, r1) dequantised on the GPU (engine/gguf.py:297-314): from
        the resident copy when there is one, else from those rows' bytes only.
        A row is n_elements / n_rows values (the reference's row_bytes), so a
        3-D tensor gives rows of its trailing dims."""
        n_rows, _ = self.row_shape(info)
        per_row = self.n_row_elements(info)
        if not (0 <= r0 <= r1 <= n_rows):
            raise ValueError(f"row range [{r0},{r1}) outside [0,{n_rows})")
        self._device_type(info)
        shape = (r1 - r0,) + info.shape[1:] if len(info.shape) > 1 else ((r1 - r0) * per_row,)
        if r1 == r0:
            return np.zeros(shape, np.float32)
        dt = self._resident.get(info.name)
        if dt is None:
            rb = self.row_bytes(info)
            dt = DeviceTensor(info, self._upload_range(info, r0 * rb, (r1 - r0) * rb))
            dt.n_rows = r1 - r0
            out = dt.rows(0, r1 - r0)
        else:
            out = dt.rows(r0, r1)
        return out.numpy().reshape(shape)

    def matmul(self, name: str, X: np.ndarray, block_rows: int = 128,
               read_once: bool = True, threads: int = 1):
        """X @ W^T for X of shape (T, in) on the GPU with W resident in HBM
        (engine/gguf.py:316-390). Returns (Y (T, out), bytes of W)."""
        info = self.tensors[name]
        n_rows, per_row = self.row_shape(info)
        Xm = np.asarray(X, dtype=np.float32)
        if Xm.ndim == 1:
            Xm = Xm[None, :]
        if Xm.shape[1] != per_row:
            raise ValueError(f"{name}: expects {per_row} inputs, got {Xm.shape[1]}")
        if info.type_id not in MATVEC_TYPES:
            raise NotImplementedError(f"no GPU matvec for {info.type_name}")
        dt = self.to_device(name)
        T = Xm.shape[0]
        x = DeviceArray.from_numpy(np.ascontiguousarray(Xm))
        y = DeviceArray.empty((T, n_rows))
        dt.matvec(x, y, T)
        return y.numpy(), info.nbytes

    def matvec(self, name: str, x: np.ndarray, block_rows: int = 64):
        """y = W @ x on the GPU (engine/gguf.py:387-417). Returns (y, bytes of W)."""
        Y, nb = self.matmul(name, np.asarray(x, dtype=np.float32)[None, :])
        return Y[0], nb
