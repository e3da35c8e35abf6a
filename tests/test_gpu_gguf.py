"""GPU parity: GGUF tensors uploaded to HBM and addressed there
(aero_gguf_upload, aero_hip_tensor_rows) against the oracle's restatement of
engine/gguf.py:232-314 (bytes, tensor, row addressing) and of the reference's
dequantisers (oracle/cpuref_quant.c, bit-identical to src/kernels.cpp).

Dequantised values are bit-exact; the device matvec over a resident weight is
within 1e-5 of the output's scale (the GEMV's bar).
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import gguf as AG
from aero_amd.device import DeviceArray as DA
from oracle import gguf_ref as G

pytestmark = pytest.mark.gpu

TYPES = (0, 1, 30, 8, 12, 13, 14, 23)     # F32 F16 BF16 Q8_0 Q4_K Q5_K Q6_K IQ4_XS


def rand_raw(rng, t, n_el):
    """Valid blocks of type t (finite fp16 scales) for n_el values."""
    from aero_amd import workloads as W
    if t == 0:
        return rng.standard_normal(n_el).astype(np.float32).tobytes()
    if t == 1:
        return rng.standard_normal(n_el).astype(np.float16).tobytes()
    if t == 30:
        return (rng.standard_normal(n_el).astype(np.float32).view(np.uint32) >> 16) \
            .astype(np.uint16).tobytes()
    bv, _bb = W.BLOCK[t]
    return W.make_table(t, n_el // bv, rng).tobytes()


def make_file(tmp_path, rng, alignment=32):
    shapes = {0: (7, 96), 1: (5, 64), 30: (9, 128), 8: (33, 96), 12: (11, 512),
              13: (6, 256), 14: (13, 256), 23: (10, 256)}
    tensors = [(f"t{t}", shapes[t], t, rand_raw(rng, t, int(np.prod(shapes[t])))) for t in TYPES]
    tensors.append(("norm", (300,), 0, rand_raw(rng, 0, 300)))
    tensors.append(("experts", (3, 4, 256), 12, rand_raw(rng, 12, 3 * 4 * 256)))
    tensors.append(("q4_0", (2, 64), 2, bytes(2 * 2 * 18)))
    data = G.write([("general.architecture", G.STRING, "llama")], tensors, alignment)
    path = tmp_path / f"m{alignment}.gguf"
    path.write_bytes(data)
    return str(path), data, G.parse(data), tensors


def oracle_rows(oracle, data, parsed, name, r0, r1):
    dims, t, _off = parsed["tensors"][name]
    raw = np.frombuffer(G.rows_bytes(data, parsed, name, r0, r1), np.uint8)
    n_el = int(np.prod(dims))
    per_row = n_el // G.row_shape(dims)[0]
    return oracle.dequant(t, raw, (r1 - r0) * per_row)


@pytest.mark.parametrize("alignment", [32, 64])
def test_tensor_and_rows_bit_exact(hip, oracle, tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    path, data, parsed, tensors = make_file(tmp_path, rng, alignment)
    with AG.GGUFReader(path) as r:
        for name, shape, t, _raw in tensors:
            if t == 2:
                continue
            info = r.tensors[name]
            n_rows, _ = G.row_shape(parsed["tensors"][name][0])
            want = oracle_rows(oracle, data, parsed, name, 0, n_rows)
            got = r.tensor(name)
            assert got.shape == shape and bits_equal(got.reshape(-1), want), name
            assert r.tensor(name) is got                  # small tensors are memoised
            for r0, r1 in ((0, 1), (1, n_rows), (n_rows // 2, n_rows), (n_rows, n_rows)):
                got_rows = r.tensor_rows(info, r0, r1)     # from those rows' bytes only
                want_rows = oracle_rows(oracle, data, parsed, name, r0, r1)
                assert bits_equal(got_rows.reshape(-1), want_rows), (name, r0, r1)
            dt = r.to_device(name)                         # resident
            assert bits_equal(dt.raw.numpy(), np.frombuffer(r.tensor_bytes(info), np.uint8))
            for r0, r1 in {(min(1, n_rows - 1), min(2, n_rows)), (0, n_rows), (n_rows - 1, n_rows)}:
                assert bits_equal(r.tensor_rows(info, r0, r1).reshape(-1),
                                  oracle_rows(oracle, data, parsed, name, r0, r1)), (name, r0, r1)
            with pytest.raises(ValueError):
                r.tensor_rows(info, 0, n_rows + 1)
        # 3-D: rows are the trailing dims
        got = r.tensor_rows(r.tensors["experts"], 1, 3)
        assert got.shape == (2, 4, 256)
        assert bits_equal(got.reshape(-1), oracle_rows(oracle, data, parsed, "experts", 1, 3))
        # a type without a GPU dequantiser is refused (its bytes stay readable)
        with pytest.raises(NotImplementedError):
            r.tensor("q4_0")
        assert r.tensor_bytes(r.tensors["q4_0"]) == bytes(72)


def test_upload_past_the_staging_chunk(hip, oracle, tmp_path):
    """A 44 MB Q4_K table (three 16 MiB staging buffers' worth, so both pinned
    buffers are reused) uploads byte for byte, also from odd byte ranges, and
    its rows gather and dequantise as the oracle's."""
    rng = np.random.default_rng(7)
    n_rows, n_per_row = 16000, 4096 + 256 * 3
    raw = rand_raw(rng, 12, n_rows * n_per_row)
    assert len(raw) > 2 * (16 << 20)
    data = G.write([("general.architecture", G.STRING, "llama")],
                   [("token_embd.weight", (n_rows, n_per_row), 12, raw)])
    path = tmp_path / "big.gguf"
    path.write_bytes(data)
    parsed = G.parse(data)
    with AG.GGUFReader(str(path)) as r:
        dt = r.to_device("token_embd.weight")
        assert bits_equal(dt.raw.numpy(), np.frombuffer(raw, np.uint8))
        from aero_amd import _lib
        L = _lib.lib()
        for b0, nb in ((3, 1000), ((16 << 20) - 5, 33), (len(raw) - 7, 7), (0, len(raw))):
            dst = DA.empty(max(nb, 1), np.uint8)
            assert L.aero_gguf_upload(r._h, b"token_embd.weight", b0, nb, dst.ptr, None) == 1
            assert dst.numpy()[:nb].tobytes() == raw[b0:b0 + nb]
        assert L.aero_gguf_upload(r._h, b"token_embd.weight", 1, len(raw), dst.ptr, None) == 0
        ids = rng.integers(0, n_rows, 37).astype(np.int32)
        out = DA.empty((37, n_per_row))
        dt.gather(DA.from_numpy(ids), out)
        table = np.frombuffer(raw, np.uint8)
        assert bits_equal(out.numpy(), oracle.embed_gather(12, table, n_rows, n_per_row, ids))
        rows = dt.rows(15990, 16000).numpy()
        assert bits_equal(rows.reshape(-1), oracle_rows(oracle, data, parsed, "token_embd.weight",
                                                        15990, 16000))


def test_resident_matvec_and_reader_matmul(hip, oracle, tmp_path):
    rng = np.random.default_rng(9)
    n_rows, n_cols = 300, 1024
    raw = rand_raw(rng, 14, n_rows * n_cols)
    data = G.write([], [("w", (n_rows, n_cols), 14, raw)])
    path = tmp_path / "w.gguf"
    path.write_bytes(data)
    X = rng.standard_normal((3, n_cols)).astype(np.float32)
    want = oracle.matmul(14, np.frombuffer(raw, np.uint8), X, n_rows)
    with AG.GGUFReader(str(path)) as r:
        Y, nb = r.matmul("w", X)
        assert nb == len(raw) and rel_to_scale(Y, want) <= RTOL
        y, _ = r.matvec("w", X[1])
        assert rel_to_scale(y, want[1]) <= RTOL
