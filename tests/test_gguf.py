"""GGUF reader: the oracle pinned, then the library's parser against it (CPU).

The oracle (oracle/gguf_ref.py) restates the reference's parse
(engine/gguf.py:186-219), row addressing (:278-314) and the C++ reader's key
lookup (src/gguf.cpp:203-218). It is pinned here by a file assembled byte by
byte from the format (every offset known), by the reference's own C++ reader
compiled from its sources (oracle/_ref/libref_gguf.so) on the same files, and
by planted mistakes. The library's parser (aero_gguf_*, through
aero_amd.gguf.GGUFReader and the C ABI) runs on the host and is checked
against the oracle and the compiled reference here; its device uploads are
GPU tests (test_gpu_gguf.py).
"""
import ctypes
import os
import struct

import numpy as np
import pytest

from aero_amd import _lib
from aero_amd import gguf as AG
from oracle import gguf_ref as G
from oracle import refbind as R

pytestmark = pytest.mark.skipif(_lib.load() is None, reason="libaero_hip.so not built")


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def rich_file(rng, alignment=32, with_u16=True):
    """Metadata of every value type (nested arrays, non-ASCII and invalid
    UTF-8 strings, an arch-scoped key shadowing a later bare key) and tensors
    of several types and shapes."""
    kv = [("general.architecture", G.STRING, "llama"),
          ("general.alignment", G.U32, alignment),
          ("llama.block_count", G.U32, 32),
          ("llama.embedding_length", G.U64, 4096),
          ("llama.rope.freq_base", G.F32, 500000.0),
          ("llama.attention.layer_norm_rms_epsilon", G.F64, 1e-5),
          ("llama.attention.head_count_kv", G.ARRAY, (G.I32, [8, 8, 4, -1])),
          ("block_count", G.U32, 7),          # shadowed by llama.block_count's suffix
          ("tokenizer.ggml.model", G.STRING, "gpt2"),
          ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["<s>", "héllo", "▁the", "日本"])),
          ("tokenizer.ggml.scores", G.ARRAY, (G.F32, [0.0, -1.5, 2.25, 3.0])),
          ("x.flags", G.ARRAY, (G.BOOL, [True, False, True])),
          ("x.nested", G.ARRAY, (G.ARRAY, [(G.U8, [1, 2]), (G.U8, [3])])),
          ("x.i8", G.I8, -5), ("x.u8", G.U8, 250), ("x.i32", G.I32, -123456),
          ("x.i64", G.I64, -(1 << 40)), ("x.bool", G.BOOL, True),
          ("x.bad_utf8", G.STRING, b"ab\xff\xfecd")]
    if with_u16:
        kv += [("x.u16", G.U16, 65000), ("x.i16", G.I16, -300)]
    tensors = []
    for name, shape, t in (("token_embd.weight", (48, 512), 12), ("output_norm.weight", (512,), 0),
                           ("blk.0.attn_q.weight", (64, 256), 8), ("blk.0.ffn_up.weight", (16, 256), 14),
                           ("blk.0.attn_norm.weight", (96,), 1), ("blk.0.x.weight", (8, 64), 30),
                           ("blk.0.y.weight", (4, 256), 23), ("blk.0.z.weight", (3, 2, 256), 13)):
        n = int(np.prod(shape))
        raw = rng.integers(0, 256, G.nbytes(t, n), dtype=np.uint8).tobytes()
        tensors.append((name, shape, t, raw))
    return kv, tensors


# ------------------------------------------------------------ the oracle

def test_oracle_parse_hand_assembled_file():
    """A file assembled from the format by hand: header 24 bytes, one u32
    metadata entry, one tensor record; the data section at the next multiple
    of 32 and the tensor's bytes there."""
    key = b"general.alignment"
    meta = struct.pack("<Q", len(key)) + key + struct.pack("<II", 4, 32)
    name = b"t"
    rec = struct.pack("<Q", 1) + name + struct.pack("<I", 2) + struct.pack("<QQ", 4, 3)
    rec += struct.pack("<I", 0) + struct.pack("<Q", 0)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
    body = head + meta + rec
    assert len(head) == 24 and len(body) == 24 + 8 + 17 + 8 + 8 + 1 + 4 + 16 + 4 + 8
    pad = (-len(body)) % 32
    payload = np.arange(12, dtype=np.float32).tobytes()
    data = body + b"\0" * pad + payload
    p = G.parse(data)
    assert p["data_offset"] == len(body) + pad == 128
    assert p["tensors"] == {"t": ((4, 3), 0, 0)}
    assert G.row_shape((4, 3)) == (3, 4)
    assert G.rows_bytes(data, p, "t", 1, 3) == payload[16:48]
    # the writer produces the same bytes for the same content (and pads the
    # file's end to the alignment, as engine/gguf.py:523 does)
    assert G.write([("general.alignment", G.U32, 32)], [("t", (3, 4), 0, payload)]) == \
        data + b"\0" * ((-len(data)) % 32)


def test_oracle_planted_mistakes_are_caught():
    """A parse that forgets the alignment padding, or that does not reverse
    the dims, disagrees with the hand-assembled layout above."""
    data = G.write([("general.alignment", G.U32, 64)],
                   [("a", (2, 32), 0, bytes(256)), ("b", (5, 32), 8, bytes(170))], alignment=64)
    p = G.parse(data)
    unpadded = 24 + (8 + 17 + 4 + 4) + 2 * (8 + 1 + 4 + 16 + 4 + 8)
    assert p["data_offset"] == 192 != unpadded
    assert p["tensors"]["b"][2] == 256          # a's 256 bytes, already a multiple of 64
    assert G.row_shape(p["tensors"]["b"][0]) == (5, 32) != (32, 5)


@pytest.mark.skipif(R.gguf() is None, reason="oracle/_ref not built")
def test_oracle_matches_compiled_reference_reader(tmp_path):
    """The reference's C++ GgufReader on the same files agrees with the oracle
    on every metadata lookup (its key map), the tensor index, sizes and data
    pointers (files without 16-bit metadata: see the next test)."""
    L = R.gguf()
    rng = np.random.default_rng(1)
    for alignment in (32, 64, 128):
        kv, tensors = rich_file(rng, alignment, with_u16=False)
        data = G.write(kv, tensors, alignment)
        path = write(tmp_path, f"f{alignment}.gguf", data)
        p = G.parse(data)
        err = ctypes.create_string_buffer(256)
        h = L.rg_open(path.encode(), err, 256)
        assert h, err.value
        try:
            assert L.rg_arch(h) == b"llama"
            assert L.rg_file_size(h) == len(data)
            look = G.cpp_lookup(p["order"], p["kv"])
            # the values as written (the C++ reader keeps string bytes as they are)
            written = G.cpp_lookup(p["order"], {kk: vv for kk, _t, vv in kv})
            for k, v in look.items():
                kb = k.encode()
                assert L.rg_has(h, kb), k
                if isinstance(v, bool) or (isinstance(v, int)):
                    assert L.rg_get_int(h, kb, -99) == int(v), k
                elif isinstance(v, float):
                    assert L.rg_get_float(h, kb, -99.0) == v, k
                elif isinstance(v, str):
                    buf = ctypes.create_string_buffer(256)
                    n = L.rg_get_str(h, kb, buf, 256)
                    want = written[k] if isinstance(written[k], bytes) else v.encode()
                    assert buf.raw[:n] == want, k
            n = L.rg_int_array(h, b"attention.head_count_kv", (ctypes.c_int64 * 8)(), 8)
            assert n == 4
            out = (ctypes.c_int64 * 4)()
            L.rg_int_array(h, b"llama.attention.head_count_kv", out, 4)
            assert list(out) == [8, 8, 4, -1]
            toks = p["kv"]["tokenizer.ggml.tokens"]
            assert L.rg_str_array_len(h, b"tokenizer.ggml.tokens") == len(toks)
            for i, tok in enumerate(toks):
                buf = ctypes.create_string_buffer(64)
                m = L.rg_str_array_item(h, b"tokenizer.ggml.tokens", i, buf, 64)
                assert buf.raw[:m].decode() == tok
            assert L.rg_n_tensors(h) == len(p["tensors"])
            ty, nd = ctypes.c_int(), ctypes.c_int()
            dims = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_int64(), ctypes.c_int64()
            for name, (d, t, o) in p["tensors"].items():
                assert L.rg_tensor(h, name.encode(), ctypes.byref(ty), ctypes.byref(nd), dims,
                                   ctypes.byref(off), ctypes.byref(nb))
                assert (ty.value, nd.value, tuple(dims[:nd.value]), off.value) == (t, len(d), d, o)
                assert nb.value == G.nbytes(t, int(np.prod(d)))
                ptr = L.rg_tensor_data(h, name.encode())
                n_rows, _ = G.row_shape(d)
                assert ctypes.string_at(ptr, nb.value) == G.rows_bytes(data, p, name, 0, n_rows)
        finally:
            L.rg_close(h)


@pytest.mark.skipif(R.gguf() is None, reason="oracle/_ref not built")
def test_reference_cpp_reader_misreads_16_bit_metadata(tmp_path):
    """Recorded difference: the reference's C++ reader reads a u16/i16 value
    as 4 bytes (src/gguf.cpp:63-64) and loses its place; the format and the
    reference's Python reader (engine/gguf.py:51-55) take 2. The oracle and the
    library follow the format."""
    data = G.write([("general.architecture", G.STRING, "llama"), ("x.u16", G.U16, 7),
                    ("x.after", G.U32, 99)], [])
    path = write(tmp_path, "u16.gguf", data)
    err = ctypes.create_string_buffer(256)
    h = R.gguf().rg_open(path.encode(), err, 256)
    if h:
        R.gguf().rg_close(h)
    assert not h and b"truncated" in err.value
    assert G.parse(data)["kv"] == {"general.architecture": "llama", "x.u16": 7, "x.after": 99}
    r = AG.GGUFReader(path)
    assert r.kv == {"general.architecture": "llama", "x.u16": 7, "x.after": 99}
    r.close()


# ------------------------------------------------------ the library's parser

def test_library_parser_matches_oracle(tmp_path):
    rng = np.random.default_rng(2)
    for alignment in (32, 64, 4096):
        kv, tensors = rich_file(rng, alignment)
        data = G.write(kv, tensors, alignment)
        path = write(tmp_path, f"r{alignment}.gguf", data)
        p = G.parse(data)
        with AG.GGUFReader(path) as r:
            assert (r.version, r.alignment, r.data_offset) == (3, alignment, p["data_offset"])
            assert r.kv == p["kv"]
            assert list(r.kv) == p["order"]
            assert r.kv_types == p["types"]
            assert r.kv["x.bad_utf8"] == "ab��cd"
            assert r.arch() == "llama" and r.hp("block_count") == 32
            assert list(r.tensors) == list(p["tensors"])
            for name, (d, t, o) in p["tensors"].items():
                info = r.tensors[name]
                n_el = int(np.prod(d))
                assert (info.dims, info.type_id, info.offset, info.n_elements) == (d, t, o, n_el)
                assert info.nbytes == G.nbytes(t, n_el)
                assert info.shape == tuple(reversed(d))
                n_rows, per_row = G.row_shape(d)
                assert r.row_shape(info) == (n_rows, per_row)
                assert r.n_row_elements(info) == n_el // n_rows
                assert r.row_bytes(info) == G.nbytes(t, n_el // n_rows)
                assert r.tensor_bytes(info) == G.rows_bytes(data, p, name, 0, n_rows)
            assert "llama" in r.summary() and "block_count = 32" in r.summary()


def test_library_c_abi_lookups_follow_the_cpp_reader(tmp_path):
    """aero_gguf_get_* take the reference C++ reader's key map: bare suffixes
    of arch keys, the first entry for a name winning (block_count -> 32, not
    the later bare key's 7), tokenizer/general keys verbatim only."""
    rng = np.random.default_rng(3)
    kv, tensors = rich_file(rng)
    data = G.write(kv, tensors)
    path = write(tmp_path, "c.gguf", data)
    p = G.parse(data)
    look = G.cpp_lookup(p["order"], p["kv"])
    L = _lib.load()
    h = L.aero_gguf_open(path.encode())
    assert h
    try:
        out = ctypes.c_int64()
        dbl = ctypes.c_double()
        n = ctypes.c_int64()
        for k, v in look.items():
            kb = k.encode()
            assert L.aero_gguf_kv_type(h, kb) >= 0, k
            if isinstance(v, bool) or isinstance(v, int):
                assert L.aero_gguf_get_int(h, kb, ctypes.byref(out)) == 1 and out.value == int(v)
            elif isinstance(v, float):
                assert L.aero_gguf_get_float(h, kb, ctypes.byref(dbl)) == 1 and dbl.value == v
            elif isinstance(v, list) and v and isinstance(v[0], str):
                assert L.aero_gguf_array_len(h, kb) == len(v)
                for i, s in enumerate(v):
                    ptr = L.aero_gguf_array_str(h, kb, i, ctypes.byref(n))
                    assert ctypes.string_at(ptr, n.value).decode() == s
        assert L.aero_gguf_get_int(h, b"block_count", ctypes.byref(out)) and out.value == 32
        assert L.aero_gguf_kv_type(h, b"ggml.model") == -1          # tokenizer keys verbatim only
        assert L.aero_gguf_kv_type(h, b"alignment") == -1           # general keys verbatim only
        vals = (ctypes.c_int64 * 4)()
        assert L.aero_gguf_array_ints(h, b"attention.head_count_kv", vals, 4) == 4
        assert list(vals) == [8, 8, 4, -1]
        ptr = L.aero_gguf_get_str(h, b"tokenizer.ggml.model", ctypes.byref(n))
        assert ctypes.string_at(ptr, n.value) == b"gpt2"
        assert L.aero_gguf_get_int(h, b"tokenizer.ggml.model", ctypes.byref(out)) == 0
        for name in p["tensors"]:
            d, t, o = p["tensors"][name]
            ptr = L.aero_gguf_tensor_data(h, name.encode())
            n_rows, _ = G.row_shape(d)
            want = G.rows_bytes(data, p, name, 0, n_rows)
            assert ctypes.string_at(ptr, len(want)) == want
        assert L.aero_gguf_tensor_info(h, b"nope", None, None, None, None, None) == -1
        assert "no tensor named nope" in _lib.last_error()
        assert L.aero_gguf_read(h, b"token_embd.weight", 0, 1 << 30, ctypes.create_string_buffer(1)) == 0
    finally:
        L.aero_gguf_close(h)


@pytest.mark.skipif(R.gguf() is None, reason="oracle/_ref not built")
def test_library_parser_matches_compiled_reference(tmp_path):
    rng = np.random.default_rng(4)
    kv, tensors = rich_file(rng, 64, with_u16=False)
    data = G.write(kv, tensors, 64)
    path = write(tmp_path, "m.gguf", data)
    Lr, L = R.gguf(), _lib.load()
    err = ctypes.create_string_buffer(256)
    hr, h = Lr.rg_open(path.encode(), err, 256), L.aero_gguf_open(path.encode())
    try:
        out = ctypes.c_int64()
        for k in ("block_count", "llama.block_count", "embedding_length", "general.alignment",
                  "x.i8", "x.u8", "x.i32", "x.i64", "x.bool"):
            assert L.aero_gguf_get_int(h, k.encode(), ctypes.byref(out)) == 1
            assert out.value == Lr.rg_get_int(hr, k.encode(), -99), k
        dbl = ctypes.c_double()
        for k in ("rope.freq_base", "attention.layer_norm_rms_epsilon"):
            assert L.aero_gguf_get_float(h, k.encode(), ctypes.byref(dbl)) == 1
            assert dbl.value == Lr.rg_get_float(hr, k.encode(), -1.0), k
        assert L.aero_gguf_n_tensors(h) == Lr.rg_n_tensors(hr)
        for name, _s, _t, _raw in tensors:
            nb = ctypes.c_int64()
            L.aero_gguf_tensor_info(h, name.encode(), None, None, None, None, ctypes.byref(nb))
            a = ctypes.string_at(L.aero_gguf_tensor_data(h, name.encode()), nb.value)
            b = ctypes.string_at(Lr.rg_tensor_data(hr, name.encode()), nb.value)
            assert a == b
    finally:
        Lr.rg_close(hr)
        L.aero_gguf_close(h)


def test_library_parser_refusals(tmp_path):
    """Each malformed file is refused with a reason (no crash, no partial
    reader): bad magic, versions 1 and 4, unknown value type, bad alignment,
    n_dims 5, non-whole blocks, tensor data past the end, element counts
    past 2^48 (including ones whose product overflows int64), and every
    truncation of a valid file."""
    good = G.write([("general.architecture", G.STRING, "llama"), ("a.b", G.U32, 1)],
                   [("t", (2, 32), 8, bytes(68))])
    cases = {
        "magic": b"GGUX" + good[4:],
        "v1": good[:4] + struct.pack("<I", 1) + good[8:],
        "v4": good[:4] + struct.pack("<I", 4) + good[8:],
        "vtype": G.write([("k", G.U32, 1)], []).replace(struct.pack("<I", 4), struct.pack("<I", 13), 1),
        "align3": G.write([("general.alignment", G.U32, 3)], [], alignment=4),
        "ndims5": G.write([], [("t", (1, 1, 1, 1, 32), 8, bytes(34))]),
        "blocks": G.write([], [("t", (1, 33), 8, bytes(68))]),
        "past_end": G.write([], [("t", (4, 32), 8, bytes(136))])[:-64],
        # element counts whose int64 product would wrap (2^80, 2^72): refused
        # before the multiply, not accepted as a small tensor
        "overflow2": G.write([], [("t", (1 << 40, 1 << 40), 0, bytes(4))]),
        "overflow3": G.write([], [("t", (1 << 24, 1 << 24, 1 << 24), 0, bytes(4))]),
    }
    for name, data in cases.items():
        path = write(tmp_path, f"bad_{name}.gguf", data)
        with pytest.raises(ValueError):
            AG.GGUFReader(path)
        assert _lib.last_error(), name
    last_byte = G.parse(good)["data_offset"] + 68     # the end of t's bytes
    for cut in range(0, last_byte, 3):
        path = write(tmp_path, "cut.gguf", good[:cut])
        with pytest.raises(ValueError):
            AG.GGUFReader(path)
    with pytest.raises(FileNotFoundError):
        AG.GGUFReader(str(tmp_path / "missing.gguf"))


def test_library_parser_large_vocabulary(tmp_path):
    """A 128k-entry token array and its scores (a Llama-3 tokenizer's size)."""
    n = 128256
    toks = [f"tok{i}Ġ" for i in range(n)]
    scores = np.linspace(-1, 1, n).astype(np.float32).tolist()
    data = G.write([("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, toks)),
                    ("tokenizer.ggml.scores", G.ARRAY, (G.F32, scores))], [])
    path = write(tmp_path, "vocab.gguf", data)
    with AG.GGUFReader(path) as r:
        assert r.kv["tokenizer.ggml.tokens"] == toks
        assert r.kv["tokenizer.ggml.scores"] == scores


def test_bench_gguf_image_matches_oracle_writer(tmp_path):
    """bench.py's GGUF image builder (the synthetic Llama-3 file of
    `bench.py --gguf`) lays out the same bytes as the oracle's writer for the
    same content, and the library's parser reads back what was written."""
    import bench

    rng = np.random.default_rng(5)
    kv, tensors = rich_file(rng, 64)
    ascii_kv = [e for e in kv if not isinstance(e[2], bytes)]
    data = bench.gguf_image(ascii_kv, [(n, s, t, raw) for n, s, t, raw in tensors], 64)
    assert data == G.write(ascii_kv, tensors, 64)
    path = write(tmp_path, "w.gguf", data)
    with AG.GGUFReader(path) as r:
        assert r.kv == G.parse(data)["kv"]
        for name, shape, t, raw in tensors:
            assert r.tensors[name].shape == shape
            assert r.tensor_bytes(r.tensors[name]) == raw
