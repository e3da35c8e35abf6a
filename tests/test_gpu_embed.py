"""GPU parity: GGUF token-embedding gather with Q8_0 / Q4_K / Q6_K dequant, and
whole-buffer dequant (F32 / F16 / BF16 too), against the oracle
(oracle/cpuref_quant.c restating src/kernels.cpp:29-73,315-458 and
src/model.cpp:297-316). Bit-exact throughout: every value is one or two IEEE
multiplies (and one subtract) in the reference's order.
"""
import numpy as np
import pytest

from conftest import bits_equal, golden
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu


def gpu_gather(e, ids=None, bad=None):
    ids = e["ids"] if ids is None else ids
    tab = DA.from_numpy(e["table"])
    dids = DA.from_numpy(ids)
    out = DA.empty((ids.size, e["n_embd"]))
    ops.embed_gather(e["type"], tab, e["vocab"], e["n_embd"], dids, out, scale=e["scale"],
                     bad_count=bad)
    return out.numpy()


@pytest.mark.parametrize("name", list(W.SHAPES))
def test_gather_layer_shapes(hip, oracle, name):
    s = W.SHAPES[name]
    e = W.embed_inputs(s)
    print(f"gather {name} type={e['type']} table={e['table'].nbytes} B ids={e['ids'].size} "
          f"scale={e['scale']}", flush=True)
    got = gpu_gather(e)
    want = oracle.embed_gather(e["type"], e["table"], e["vocab"], e["n_embd"], e["ids"],
                               e["scale"])
    assert bits_equal(got, want)


def test_gather_edge_ids_and_bad_count(hip, oracle):
    s = W.SHAPES["qwen2_0p5b_decode"]
    e = W.embed_inputs(s, vocab=1000, rows=4)
    ids = np.array([0, 999, -1, 1000, 5, 2**31 - 1, 999], np.int32)
    bad = DA.from_numpy(np.zeros(1, np.uint32))
    got = gpu_gather(e, ids=ids, bad=bad)
    assert int(bad.numpy()[0]) == 3
    for r in (2, 3, 5):
        assert not got[r].any()
    ok = [0, 1, 4, 6]
    want = oracle.embed_gather(e["type"], e["table"], 1000, s.hidden, ids[ok])
    assert bits_equal(got[ok], want)


@pytest.mark.parametrize("t", [W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS])
def test_gather_brute_force_rows(hip, oracle, t):
    """Row selection: each output row equals the dequant of exactly that table row."""
    rng = np.random.default_rng(t)
    bv, bb = W.BLOCK[t]
    n_embd, vocab = 2 * bv, 37
    table = W.make_table(t, vocab * 2, rng)
    ids = rng.integers(0, vocab, 50).astype(np.int32)
    e = {"type": t, "table": table, "vocab": vocab, "n_embd": n_embd, "ids": ids, "scale": 0.0}
    got = gpu_gather(e)
    rb = 2 * bb
    for i, tok in enumerate(ids):
        row = oracle.dequant(t, table[tok * rb:(tok + 1) * rb], n_embd)
        assert bits_equal(got[i], row)


@pytest.mark.parametrize("t,n_embd,rows", [
    (W.Q8_0, 32 * 45, 32768),    # 2-byte aligned odd rows, runs of 4 steps, ragged tail
    (W.Q6_K, 256 * 5, 40000),    # 2-byte aligned odd rows, runs of 4 steps, one-block tail
    (W.Q4_K, 256 * 48, 8192),    # runs of 8 steps
    (W.Q5_K, 256 * 16, 16384),   # runs of 4 steps (over 64K steps)
    (W.IQ4_XS, 256 * 10, 3000),  # whole-row runs of 16 steps
    (W.Q8_0, 32 * 7, 3),         # a row shorter than one 256-value step
])
def test_gather_run_lengths(hip, oracle, t, n_embd, rows):
    """Long gathers take multi-step runs per wave; row lengths that are not a
    whole number of runs, and rows that start 2 bytes past a 4-byte boundary,
    still select and decode every value exactly. Some ids are out of range."""
    rng = np.random.default_rng(n_embd + rows)
    bv, bb = W.BLOCK[t]
    vocab = 997
    table = W.make_table(t, vocab * (n_embd // bv), rng)
    ids = rng.integers(0, vocab, rows).astype(np.int32)
    ids[::1009] = -5
    ids[7::2003] = vocab
    n_bad = int(((ids < 0) | (ids >= vocab)).sum())
    print(f"gather runs type={t} n_embd={n_embd} rows={rows} bad={n_bad}", flush=True)
    bad = DA.from_numpy(np.zeros(1, np.uint32))
    e = {"type": t, "table": table, "vocab": vocab, "n_embd": n_embd, "ids": ids, "scale": 0.0}
    got = gpu_gather(e, bad=bad)
    assert int(bad.numpy()[0]) == n_bad
    ok = (ids >= 0) & (ids < vocab)
    assert not got[~ok].any()
    want = oracle.embed_gather(t, table, vocab, n_embd, ids[ok])
    assert bits_equal(got[ok], want)


def test_dequant_types(hip, oracle):
    rng = np.random.default_rng(31)
    cases = [(W.F32, 4, 1), (W.F16, 2, 1), (W.BF16, 2, 1), (W.Q8_0, 34, 32), (W.Q4_K, 144, 256),
             (W.Q5_K, 176, 256), (W.Q6_K, 210, 256), (W.IQ4_XS, 136, 256)]
    for t, bb, bv in cases:
        nb = 1001
        if t in W.BLOCK:
            raw = W.make_table(t, nb, rng)
        else:
            raw = rng.integers(0, 256, nb * bb, dtype=np.uint8)
        n = nb * bv
        out = DA.empty(n)
        ops.dequant(t, DA.from_numpy(raw), out, n)
        assert bits_equal(out.numpy(), oracle.dequant(t, raw, n)), t


def test_f16_exhaustive(hip):
    """All 65536 half patterns (subnormals, inf, NaN payloads) decode exactly."""
    h = np.arange(65536, dtype=np.uint16)
    out = DA.empty(65536)
    ops.dequant(W.F16, DA.from_numpy(h.view(np.uint8)), out, 65536)
    assert np.array_equal(out.numpy().view(np.uint32),
                          h.view(np.float16).astype(np.float32).view(np.uint32))


def test_q8_0_subnormal_scales(hip, oracle):
    """fp16 d below 6.1e-5 (subnormal) in Q8_0 blocks: still bit-exact."""
    rng = np.random.default_rng(32)
    nb = 4096
    blk = np.empty((nb, 34), np.uint8)
    d = (np.arange(nb) % 1024 + 1).astype(np.uint16)  # every subnormal mantissa
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    raw = blk.reshape(-1)
    out = DA.empty(nb * 32)
    ops.dequant(W.Q8_0, DA.from_numpy(raw), out, nb * 32)
    assert bits_equal(out.numpy(), oracle.dequant(W.Q8_0, raw, nb * 32))


def test_dequant_kat(hip):
    k = golden("kat_quant.npz")
    for name, t in (("q4k_nibbles", W.Q4_K), ("q4k_pack_dmin0", W.Q4_K),
                    ("q4k_pack_dmin1", W.Q4_K), ("q6k_zero", W.Q6_K), ("q6k_ones", W.Q6_K),
                    ("q6k_lownib", W.Q6_K), ("q8_0_ramp", W.Q8_0)):
        raw, want = k[name + "_raw"], k[name + "_want"]
        out = DA.empty(want.size)
        ops.dequant(t, DA.from_numpy(raw), out, want.size)
        assert bits_equal(out.numpy(), want), name
    raw = k["q4k_nibbles_dmin2_raw"]
    out = DA.empty(256)
    ops.dequant(W.Q4_K, DA.from_numpy(raw), out, 256)
    assert bits_equal(out.numpy(), k["q4k_nibbles_want"])


def test_dequant_golden(hip):
    g = golden("ref_vectors.npz")
    for t, bv in ((8, 32), (12, 256), (13, 256), (14, 256), (23, 256)):
        raw = g[f"deq{t}_raw"]
        want = g[f"deq{t}_out"]
        out = DA.empty(want.size)
        ops.dequant(t, DA.from_numpy(raw), out, want.size)
        assert bits_equal(out.numpy(), want), t
