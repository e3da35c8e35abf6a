"""GGUF parse, row addressing and a fixture writer, restated from the reference.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Plain-Python restatement of
- the parse of engine/gguf.py:186-219 (GGUFReader._parse_index): header, the
  metadata dict (scalars at their natural width, strings decoded as UTF-8 with
  replacement, arrays as lists), the tensor index and the data section at the
  next multiple of general.alignment (default 32, a power of two);
- the byte sizes of engine/quant.py:ggml_type_size and the row addressing of
  engine/gguf.py:278-314 (row_bytes, row_shape, the bytes of rows [r0, r1));
- the key lookup of the reference's C++ reader, src/gguf.cpp:203-218 (every
  key, and the part after its first dot unless the key starts with
  "tokenizer" or "general."; the first entry for a name wins);
- a writer with the layout of engine/gguf.py:448-526 (GGUFWriter): version
  3, metadata, tensor index, each tensor's data at a multiple of the
  alignment, for fixtures.
"""
from __future__ import annotations

import struct
from typing import Any, Dict, List, Tuple

MAGIC = b"GGUF"
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

# ggml type -> (values, bytes) per block (src/gguf.cpp:106-139)
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
         8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 23: (256, 136)}


class _Cur:
    def __init__(self, b: bytes):
        self.b, self.p = b, 0

    def take(self, n: int) -> bytes:
        if self.p + n > len(self.b):
            raise EOFError("truncated")
        s = self.b[self.p:self.p + n]
        self.p += n
        return s

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def s(self) -> str:
        return self.take(self.u64()).decode("utf-8", "replace")

    def value(self, t: int) -> Any:
        if t == STRING:
            return self.s()
        if t == ARRAY:
            et, n = self.u32(), self.u64()
            return [self.value(et) for _ in range(n)]
        f = _FMT.get(t)
        if f is None:
            raise ValueError(f"unknown GGUF value type {t}")
        return struct.unpack(f, self.take(struct.calcsize(f)))[0]


def parse(data: bytes) -> Dict[str, Any]:
    """engine/gguf.py:186-219 on the file's bytes."""
    c = _Cur(data)
    if c.take(4) != MAGIC:
        raise ValueError("bad magic")
    version = c.u32()
    if version not in (2, 3):
        raise ValueError(f"unsupported GGUF version {version}")
    n_tensors, n_kv = c.u64(), c.u64()
    kv: Dict[str, Any] = {}
    types: Dict[str, int] = {}
    order: List[str] = []
    for _ in range(n_kv):
        key = c.s()
        t = c.u32()
        kv[key] = c.value(t)
        types[key] = t
        order.append(key)
    alignment = int(kv.get("general.alignment", 32))
    if alignment <= 0 or alignment & (alignment - 1):
        raise ValueError(f"bad alignment {alignment}")
    tensors: Dict[str, Tuple[Tuple[int, ...], int, int]] = {}
    for _ in range(n_tensors):
        name = c.s()
        nd = c.u32()
        dims = tuple(c.u64() for _ in range(nd))
        t = c.u32()
        off = c.u64()
        tensors[name] = (dims, t, off)
    data_offset = c.p + (-c.p) % alignment
    return {"version": version, "kv": kv, "types": types, "order": order,
            "alignment": alignment, "tensors": tensors, "data_offset": data_offset}


def cpp_lookup(order: List[str], kv: Dict[str, Any]) -> Dict[str, Any]:
    """The C++ reader's key map (src/gguf.cpp:203-218): first entry wins."""
    m: Dict[str, Any] = {}
    for key in order:
        dot = key.find(".")
        if dot >= 0 and not key.startswith("tokenizer") and not key.startswith("general."):
            m.setdefault(key[dot + 1:], kv[key])
        m.setdefault(key, kv[key])
    return m


def nbytes(type_id: int, n_elements: int) -> int:
    bv, bb = BLOCK[type_id]
    if n_elements % bv:
        raise ValueError("not whole blocks")
    return n_elements // bv * bb


def row_shape(dims: Tuple[int, ...]) -> Tuple[int, int]:
    """engine/gguf.py:290-295 (shape = dims reversed; 1-D is one row)."""
    shape = tuple(reversed(dims))
    if len(shape) <= 1:
        return 1, int(shape[0]) if shape else 0
    return int(shape[0]), int(shape[1])


def rows_bytes(data: bytes, parsed: Dict[str, Any], name: str, r0: int, r1: int) -> bytes:
    """The file bytes of rows [r0, r1) (engine/gguf.py:297-314 before dequant).
    A row is n_elements / n_rows values, the reference's row_bytes
    (:278-288); for 1-D and 2-D tensors that is row_shape's n_per_row, which
    the reference's tensor_rows uses (for 3-D it takes shape[1] and fails)."""
    dims, t, off = parsed["tensors"][name]
    n_rows, _ = row_shape(dims)
    if not (0 <= r0 <= r1 <= n_rows):
        raise ValueError(f"row range [{r0},{r1}) outside [0,{n_rows})")
    n_el = 1
    for d in dims:
        n_el *= d
    rb = nbytes(t, n_el // n_rows)
    start = parsed["data_offset"] + off + r0 * rb
    return data[start:start + (r1 - r0) * rb]


def _w_str(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _w_value(t: int, v: Any) -> bytes:
    if t == STRING:
        return _w_str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_w_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write(kv: List[Tuple[str, int, Any]], tensors: List[Tuple[str, Tuple[int, ...], int, bytes]],
          alignment: int = 32, version: int = 3) -> bytes:
    """A GGUF file (engine/gguf.py:483-526 layout). tensors: (name, row-major
    shape, ggml type, raw bytes); each tensor's data starts at a multiple of
    `alignment` in the data section."""
    out = bytearray(MAGIC)
    out += struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        out += _w_str(key) + struct.pack("<I", t) + _w_value(t, v)
    offsets, cur = [], 0
    for _n, _s, _t, raw in tensors:
        offsets.append(cur)
        cur += len(raw)
        cur += (-cur) % alignment
    for (name, shape, t, _raw), off in zip(tensors, offsets):
        dims = tuple(reversed(shape))
        out += _w_str(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", t, off)
    out += b"\x00" * ((-len(out)) % alignment)
    start = len(out)
    for (_n, _s, _t, raw), off in zip(tensors, offsets):
        out += b"\x00" * (start + off - len(out))
        out += raw
    out += b"\x00" * ((-len(out)) % alignment)
    return bytes(out)
