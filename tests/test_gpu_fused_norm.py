"""GPU parity: the two norms fused along the model loop's data flow, against
the oracle's composition of the steps they replace.

* embed_rmsnorm: the embedding gather (src/model.cpp:297-316) followed by the
  first block's RMSNorm (src/model.cpp:244-245). x is bit-exact against the
  oracle's gather; h within 1e-5 of scale against the oracle's rmsnorm_rows
  of that x.
* add_rmsnorm: the residual add `x_ += o_` followed by norm_row
  (src/model.cpp:279-282). x + d is bit-exact (one IEEE add); h within 1e-5
  of scale against the oracle's rmsnorm_rows of the sum.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import _lib, ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu


def norm_weight(s, rng):
    if s.unit_offset:
        return rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1)
    return np.float32(1) + rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1)


def gpu_embed_norm(e, w, eps, unit_offset, ids=None, bad=None):
    ids = e["ids"] if ids is None else ids
    tab = DA.from_numpy(e["table"])
    dids = DA.from_numpy(ids)
    x = DA.empty((ids.size, e["n_embd"]))
    h = DA.empty((ids.size, e["n_embd"]))
    ops.embed_rmsnorm(e["type"], tab, e["vocab"], e["n_embd"], dids, x, h,
                      None if w is None else DA.from_numpy(w), eps, scale=e["scale"],
                      unit_offset=unit_offset, bad_count=bad)
    return x.numpy(), h.numpy()


@pytest.mark.parametrize("name", list(W.SHAPES))
def test_embed_rmsnorm_layer_shapes(hip, oracle, name):
    s = W.SHAPES[name]
    e = W.embed_inputs(s)
    w = norm_weight(s, np.random.default_rng(1))
    print(f"embed_rmsnorm {name} type={e['type']} rows={e['ids'].size} n={s.hidden} "
          f"scale={e['scale']} unit_offset={s.unit_offset}", flush=True)
    x, h = gpu_embed_norm(e, w, s.eps, s.unit_offset)
    want_x = oracle.embed_gather(e["type"], e["table"], e["vocab"], e["n_embd"], e["ids"],
                                 e["scale"])
    assert bits_equal(x, want_x)
    want_h = oracle.rmsnorm_rows(want_x, w, s.eps, s.unit_offset)
    assert rel_to_scale(h, want_h) <= RTOL


@pytest.mark.parametrize("t", [W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS])
@pytest.mark.parametrize("n_blocks_row", [1, 3, 7, 16, 45])
def test_embed_rmsnorm_types_and_widths(hip, oracle, t, n_blocks_row):
    """Every block type at row widths that leave a short last step or idle
    waves, rows starting 2 bytes past a 4-byte boundary (odd Q8_0 / Q6_K
    rows), weightless and (1+w) forms."""
    rng = np.random.default_rng(100 * t + n_blocks_row)
    bv, bb = W.BLOCK[t]
    n_embd, vocab = n_blocks_row * bv, 61
    table = W.make_table(t, vocab * n_blocks_row, rng)
    ids = rng.integers(0, vocab, 37).astype(np.int32)
    e = {"type": t, "table": table, "vocab": vocab, "n_embd": n_embd, "ids": ids, "scale": 0.0}
    want_x = oracle.embed_gather(t, table, vocab, n_embd, ids)
    for w, uo in ((None, False), (rng.standard_normal(n_embd, dtype=np.float32), True)):
        x, h = gpu_embed_norm(e, w, 1e-6, uo)
        assert bits_equal(x, want_x)
        assert rel_to_scale(h, oracle.rmsnorm_rows(want_x, w, 1e-6, uo)) <= RTOL


def test_embed_rmsnorm_bad_ids(hip, oracle):
    s = W.SHAPES["qwen2_0p5b_decode"]
    e = W.embed_inputs(s, vocab=1000, rows=4)
    ids = np.array([0, 999, -1, 1000, 5, 2**31 - 1, 999], np.int32)
    bad = DA.from_numpy(np.zeros(1, np.uint32))
    w = norm_weight(s, np.random.default_rng(2))
    x, h = gpu_embed_norm(e, w, s.eps, False, ids=ids, bad=bad)
    assert int(bad.numpy()[0]) == 3
    for r in (2, 3, 5):
        assert not x[r].any() and not h[r].any()
    ok = [0, 1, 4, 6]
    want_x = oracle.embed_gather(e["type"], e["table"], 1000, s.hidden, ids[ok])
    assert bits_equal(x[ok], want_x)
    assert rel_to_scale(h[ok], oracle.rmsnorm_rows(want_x, w, s.eps)) <= RTOL


def test_embed_rmsnorm_refusals(hip):
    """Refused on the host, before any launch: a row wider than 8 waves of 8
    steps, x_out == h_out, a misaligned weight."""
    rng = np.random.default_rng(3)
    t = W.Q4_K
    table = DA.from_numpy(W.make_table(t, 2 * 65, rng))
    ids = DA.from_numpy(np.zeros(1, np.int32))
    x = DA.empty((1, 65 * 256))
    h = DA.empty((1, 65 * 256))
    L = _lib.lib()
    assert L.aero_hip_embed_rmsnorm(t, table.ptr, table.nbytes, 2, 65 * 256, ids.ptr, 1, 0.0,
                                    x.ptr, None, 1e-6, 0, h.ptr, None, None) == 0
    assert "waves" in _lib.last_error()
    assert L.aero_hip_embed_rmsnorm(t, table.ptr, table.nbytes, 2, 256, ids.ptr, 1, 0.0,
                                    x.ptr, None, 1e-6, 0, x.ptr, None, None) == 0
    w = DA.empty((257,))
    assert L.aero_hip_embed_rmsnorm(t, table.ptr, table.nbytes, 2, 256, ids.ptr, 1, 0.0,
                                    x.ptr, w.ptr + 4, 1e-6, 0, h.ptr, None, None) == 0


# ------------------------------------------------------------ add_rmsnorm
def add_inputs(s, seed=0, rows=None):
    rng = np.random.default_rng(seed)
    R = s.n_tok if rows is None else rows
    x = rng.standard_normal((R, s.hidden), dtype=np.float32)
    d = rng.standard_normal((R, s.hidden), dtype=np.float32)
    return x, d, norm_weight(s, rng)


@pytest.mark.parametrize("name", list(W.SHAPES))
def test_add_rmsnorm_layer_shapes(hip, oracle, name):
    s = W.SHAPES[name]
    x, d, w = add_inputs(s)
    print(f"add_rmsnorm {name} rows={x.shape[0]} n={s.hidden} unit_offset={s.unit_offset}",
          flush=True)
    dx, dd, dw = DA.from_numpy(x), DA.from_numpy(d), DA.from_numpy(w)
    h = DA.empty(x.shape)
    ops.add_rmsnorm(dx, dd, dw, h, x.shape[0], s.hidden, s.eps, s.unit_offset)
    want_x = x + d
    assert bits_equal(dx.numpy(), want_x)          # in place, as the reference
    assert bits_equal(dd.numpy(), d)
    assert rel_to_scale(h.numpy(), oracle.rmsnorm_rows(want_x, w, s.eps, s.unit_offset)) <= RTOL


@pytest.mark.parametrize("rows,cols", [(1, 4), (3, 896), (5, 1001), (7, 4098), (2, 8192 * 4),
                                       (64, 6)])
@pytest.mark.parametrize("form", ["in_place", "out_of_place", "into_d", "weightless"])
def test_add_rmsnorm_forms(hip, oracle, rows, cols, form):
    """Vector and scalar kernels (cols not a multiple of 4, rows wider than
    one workgroup's registers), x_out in place / separate / over d, no weight."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    d = rng.standard_normal((rows, cols), dtype=np.float32)
    w = None if form == "weightless" else rng.standard_normal(cols, dtype=np.float32)
    dx, dd = DA.from_numpy(x), DA.from_numpy(d)
    h = DA.empty(x.shape)
    xo = {"in_place": None, "weightless": None, "out_of_place": DA.empty(x.shape),
          "into_d": dd}[form]
    ops.add_rmsnorm(dx, dd, None if w is None else DA.from_numpy(w), h, rows, cols, 1e-5,
                    x_out=xo)
    want_x = x + d
    got_x = (dx if xo is None else xo).numpy()
    assert bits_equal(got_x, want_x)
    if form == "out_of_place":
        assert bits_equal(dx.numpy(), x)
    assert rel_to_scale(h.numpy(), oracle.rmsnorm_rows(want_x, w, 1e-5)) <= RTOL


def test_add_rmsnorm_refuses_aliased_h(hip):
    x = DA.empty((2, 64))
    d = DA.empty((2, 64))
    L = _lib.lib()
    for h in (x, d):
        assert L.aero_hip_add_rmsnorm(x.ptr, d.ptr, x.ptr, None, h.ptr, 2, 64, 1e-6, 0,
                                      None) == 0
    assert L.aero_hip_add_rmsnorm(x.ptr, d.ptr, x.ptr, None, d.ptr, 2, 64, 1e-6,
                                  ops.NORM_L2, None) == 0


# ------------------------------------------------------------ post_norm_add
def post_norm_ref(oracle, y, x, w1, w2, eps, ds, ss, unit):
    """The reference's gemma_block site (src/model.cpp:213-219, 228-231):
    a = norm_row(y, w1); x' = (x + ds*a) * ss; h = norm_row(x', w2)."""
    a = oracle.rmsnorm_rows(y, w1, eps, unit)
    xn = ((x + np.float32(ds) * a) * np.float32(ss)).astype(np.float32)
    return xn, oracle.rmsnorm_rows(xn, w2, eps, unit)


@pytest.mark.parametrize("rows,cols", [(2048, 2560), (64, 2560), (1, 2560), (512, 4096),
                                       (7, 8192), (33, 1000), (5, 130)])
@pytest.mark.parametrize("ds,ss", [(1.0, 1.0), (0.7, 1.0), (1.0, 1.3), (0.5, 0.9)])
@pytest.mark.parametrize("unit", [False, True])
def test_post_norm_add_vs_oracle(hip, oracle, rows, cols, ds, ss, unit):
    """x' within one rounding of every step (the post-norm's 1e-5 carried
    through the add) and h within 1e-5 of scale of the oracle's composition;
    the Gemma-3-4B-style config-3 shape (2048 x 2560) among them."""
    rng = np.random.default_rng(rows * cols)
    y = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(3)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    w1 = (rng.standard_normal(cols) * 0.1 + (0 if unit else 1)).astype(np.float32)
    w2 = (rng.standard_normal(cols) * 0.1 + (0 if unit else 1)).astype(np.float32)
    print(f"post_norm_add {rows}x{cols} ds={ds} ss={ss} unit={unit}", flush=True)
    dy, dx = DA.from_numpy(y), DA.from_numpy(x)
    h = DA.empty((rows, cols))
    ops.post_norm_add(dy, dx, DA.from_numpy(w1), DA.from_numpy(w2), h, rows, cols, 1e-6,
                      ds=ds, ss=ss, unit_offset=unit)
    want_x, want_h = post_norm_ref(oracle, y, x, w1, w2, 1e-6, ds, ss, unit)
    assert rel_to_scale(dx.numpy(), want_x) <= RTOL
    assert rel_to_scale(h.numpy(), want_h) <= RTOL


def test_post_norm_add_out_of_place_and_weightless(hip, oracle):
    rng = np.random.default_rng(3)
    y = rng.standard_normal((40, 2560), dtype=np.float32)
    x = rng.standard_normal((40, 2560), dtype=np.float32)
    dy, dx, xo, h = DA.from_numpy(y), DA.from_numpy(x), DA.empty((40, 2560)), DA.empty((40, 2560))
    ops.post_norm_add(dy, dx, None, None, h, 40, 2560, 1e-6, ds=0.8, x_out=xo)
    want_x, want_h = post_norm_ref(oracle, y, x, None, None, 1e-6, 0.8, 1.0, False)
    assert bits_equal(dx.numpy(), x)                      # x untouched
    assert rel_to_scale(xo.numpy(), want_x) <= RTOL
    assert rel_to_scale(h.numpy(), want_h) <= RTOL


def test_post_norm_add_refusals(hip):
    a, b, c = DA.empty((4, 64)), DA.empty((4, 64)), DA.empty((4, 64))
    for args in ((a, b, None, None, a), (a, b, None, None, b)):
        with pytest.raises(_lib.AeroHipError, match="alias"):
            ops.post_norm_add(*args, 4, 64, 1e-6)
    with pytest.raises(_lib.AeroHipError, match="alias"):
        ops.post_norm_add(a, b, None, None, c, 4, 64, 1e-6, x_out=a)
