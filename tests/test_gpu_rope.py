"""GPU parity: fused per-head RMSNorm -> RoPE (and plain RoPE) against the
oracle's composition of src/attention_layer.cpp:89-156 (per-head rmsnorm,
rope_tables, apply_rope), at the layer shapes and at edge shapes.

With a pre-computed table the GPU does the reference's arithmetic on the same
cos/sin values, so the result is bit-exact. With computed angles the fp32
angle is bit-identical ((float)pos * inv, inv from the host) and only the
sin/cos implementations differ (ulp level): RTOL applies.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, golden, rel_to_scale
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu


def gpu_rope(q, pos, head_dim, n_rot, *, k=None, theta=1e4, mode=0, q_w=None, k_w=None,
             eps=1e-6, unit_offset=False, table=None, out_of_place=False, ff=None):
    T = q.shape[0]
    hq = q.size // (T * head_dim)
    hk = 0 if k is None else k.size // (T * head_dim)
    dq = DA.from_numpy(q)
    dk = None if k is None else DA.from_numpy(k)
    qo = DA.empty(q.shape) if out_of_place else None
    ko = DA.empty(k.shape) if (out_of_place and k is not None) else None
    kw = {}
    if n_rot < 2:
        pass
    elif table is None:
        n, inv = ops.rope_inv_freq(n_rot, n_rot, theta, ff)
        kw["inv_freq"] = DA.from_numpy(inv)
    else:
        kw["cos_tab"] = DA.from_numpy(table[0])
        kw["sin_tab"] = DA.from_numpy(table[1])
    ops.qk_norm_rope(dq, hq, T, head_dim, n_rot, k=dk, n_k_heads=hk, q_out=qo, k_out=ko,
                     q_norm_w=None if q_w is None else DA.from_numpy(q_w),
                     k_norm_w=None if k_w is None else DA.from_numpy(k_w), eps=eps,
                     unit_offset=unit_offset, mode=mode, pos=DA.from_numpy(pos), **kw)
    rq = (qo or dq).numpy()
    rk = None if k is None else (ko or dk).numpy()
    return rq, rk


def oracle_rope(oracle, x, pos, head_dim, n_rot, theta=1e4, mode=0, w=None, eps=1e-6,
                unit_offset=False, table=None, ff=None):
    T = x.shape[0]
    H = x.size // (T * head_dim)
    if table is None:
        return oracle.qk_norm_rope(x, T, H, head_dim, n_rot, pos, theta, mode, w, eps,
                                   unit_offset, ff)
    return oracle.qk_norm_rope(x, T, H, head_dim, n_rot, pos, theta, mode, w, eps,
                               unit_offset, cos_tab=table[0], sin_tab=table[1])


@pytest.mark.parametrize("name", ["qwen2_0p5b_decode", "llama3_8b_prefill", "gemma3_4b_prefill",
                                  "qwen3next_hybrid"])
def test_rope_layer_shapes_computed_angle(hip, oracle, name):
    s = W.SHAPES[name]
    d = W.rope_inputs(s)
    print(f"rope {name} q{d['q'].shape} k{d['k'].shape} n_rot={s.n_rot} "
          f"norm={'q_w' in d}", flush=True)
    gq, gk = gpu_rope(d["q"], d["pos"], s.head_dim, s.n_rot, k=d["k"], theta=s.theta,
                      q_w=d.get("q_w"), k_w=d.get("k_w"), eps=s.eps, unit_offset=s.unit_offset)
    wq = oracle_rope(oracle, d["q"], d["pos"], s.head_dim, s.n_rot, s.theta, 0, d.get("q_w"),
                     s.eps, s.unit_offset)
    wk = oracle_rope(oracle, d["k"], d["pos"], s.head_dim, s.n_rot, s.theta, 0, d.get("k_w"),
                     s.eps, s.unit_offset)
    assert rel_to_scale(gq, wq) <= RTOL
    assert rel_to_scale(gk, wk) <= RTOL
    if s.n_rot < s.head_dim and "q_w" not in d:
        # in-place partial rotation leaves the tail channels bit-identical
        assert bits_equal(gq[..., s.n_rot:], d["q"][..., s.n_rot:])


@pytest.mark.parametrize("name", ["llama3_70b_decode64", "llama3_70b_prefill16k"])
def test_rope_layer_shapes_table(hip, oracle, name):
    s = W.SHAPES[name]
    d = W.rope_inputs(s)
    cos, sin = oracle.rope_tables(s.head_dim, np.arange(s.rope_table, dtype=np.int32), s.theta)
    print(f"rope-table {name} q{d['q'].shape} table {cos.shape}", flush=True)
    gq, gk = gpu_rope(d["q"], d["pos"], s.head_dim, s.n_rot, k=d["k"], table=(cos, sin))
    # every token against the oracle, in slices of 2048 tokens; same table,
    # same operation order: bit-exact
    for t0 in range(0, s.n_tok, 2048):
        rows = slice(t0, min(s.n_tok, t0 + 2048))
        wq = oracle_rope(oracle, d["q"][rows], d["pos"][rows], s.head_dim, s.n_rot,
                         table=(cos, sin))
        wk = oracle_rope(oracle, d["k"][rows], d["pos"][rows], s.head_dim, s.n_rot,
                         table=(cos, sin))
        assert bits_equal(gq[rows], wq), f"q tokens {rows}"
        assert bits_equal(gk[rows], wk), f"k tokens {rows}"
    # and every head row's norm is preserved
    nq = np.linalg.norm(gq.astype(np.float64), axis=-1)
    n0 = np.linalg.norm(d["q"].astype(np.float64), axis=-1)
    assert np.abs(nq - n0).max() / n0.max() < 1e-5


@pytest.mark.parametrize("D,n_rot,mode,norm,oop", [
    (16, 16, 0, False, False), (16, 16, 1, False, False), (16, 8, 0, False, False),
    (32, 8, 1, False, True), (64, 64, 1, True, False), (64, 32, 0, True, True),
    (128, 128, 1, True, True), (256, 64, 0, True, False), (256, 256, 1, False, True),
    (512, 512, 0, True, False), (512, 128, 1, False, False), (128, 48, 0, True, False),
    (128, 0, 0, True, False)])
def test_rope_variants(hip, oracle, D, n_rot, mode, norm, oop):
    rng = np.random.default_rng(D * 7 + n_rot + mode)
    T, H, HK = 9, 3, 2
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, HK, D)).astype(np.float32)
    pos = rng.integers(0, 3000, T).astype(np.int32)
    qw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    kw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    gq, gk = gpu_rope(q, pos, D, n_rot, k=k, theta=1e4, mode=mode, q_w=qw, k_w=kw,
                      out_of_place=oop)
    wq = oracle_rope(oracle, q, pos, D, n_rot, 1e4, mode, qw)
    wk = oracle_rope(oracle, k, pos, D, n_rot, 1e4, mode, kw)
    assert rel_to_scale(gq, wq) <= RTOL
    assert rel_to_scale(gk, wk) <= RTOL


@pytest.mark.parametrize("mode,n_rot,norm,oop,table", [
    (0, 64, False, False, False), (1, 64, True, False, False), (0, 32, True, False, False),
    (1, 16, False, True, False), (0, 16, False, False, False), (1, 32, False, False, True),
    (0, 64, True, False, True)])
def test_rope_token_tiles(hip, oracle, mode, n_rot, norm, oop, table):
    """Long inputs are processed in tiles of several tokens per workgroup (the
    cos/sin of each token of the tile in LDS): 16411 tokens leave a ragged last
    tile; with a table, tokens whose position is outside it sit inside tiles
    and must be left untouched while their neighbours are rotated."""
    rng = np.random.default_rng(1000 + 10 * n_rot + mode)
    T, H, HK, D = 16411, 5, 1, 64
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, HK, D)).astype(np.float32)
    pos = rng.integers(0, 4096, T).astype(np.int32)
    tab = None
    bad = np.zeros(T, bool)
    if table:
        tab = oracle.rope_tables(n_rot, np.arange(4000, dtype=np.int32), 1e4)
        bad = pos >= 4000
        pos[::997] = -3
        bad[::997] = True
    qw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    kw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    print(f"rope tiles T={T} mode={mode} n_rot={n_rot} norm={norm} oop={oop} table={table} "
          f"bad={int(bad.sum())}", flush=True)
    gq, gk = gpu_rope(q, pos, D, n_rot, k=k, theta=1e4, mode=mode, q_w=qw, k_w=kw,
                      out_of_place=oop, table=tab)
    ok = ~bad
    wq = oracle_rope(oracle, q[ok], pos[ok], D, n_rot, 1e4, mode, qw, table=tab)
    wk = oracle_rope(oracle, k[ok], pos[ok], D, n_rot, 1e4, mode, kw, table=tab)
    if table and not norm:  # same cos/sin, same operations: bit-exact
        assert bits_equal(gq[ok], wq) and bits_equal(gk[ok], wk)
    else:  # computed angles, or the norm's tree sum of squares
        assert rel_to_scale(gq[ok], wq) <= RTOL
        assert rel_to_scale(gk[ok], wk) <= RTOL
    if table and not oop:
        assert bits_equal(gq[bad], q[bad]) and bits_equal(gk[bad], k[bad])


@pytest.mark.parametrize("D,n_rot", [(80, 80), (80, 32), (6, 4), (10, 6), (24, 12), (64, 63)])
def test_rope_generic_kernel(hip, oracle, D, n_rot):
    """Shapes outside the vector kernel (D or n_rot not a multiple of 8, or
    D/8 not a power of two) take the one-wave-per-row kernel."""
    rng = np.random.default_rng(D + 100 * n_rot)
    T, H = 5, 3
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.arange(T, dtype=np.int32) * 7
    for norm in (False, True):
        w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
        for mode in (0, 1):
            gq, _ = gpu_rope(q, pos, D, n_rot, mode=mode, q_w=w)
            wq = oracle_rope(oracle, q, pos, D, n_rot - n_rot % 2, 1e4, mode, w)
            assert rel_to_scale(gq, wq) <= RTOL, (norm, mode)


def test_rope_q_only_and_freq_factors(hip, oracle):
    rng = np.random.default_rng(21)
    T, H, D = 7, 4, 64
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = rng.integers(0, 500, T).astype(np.int32)
    ff = np.concatenate([np.ones(16, np.float32), np.full(16, 1e30, np.float32)])
    gq, _ = gpu_rope(q, pos, D, D, theta=1e4, ff=ff)
    wq = oracle_rope(oracle, q, pos, D, D, 1e4, ff=ff)
    assert rel_to_scale(gq, wq) <= RTOL
    # pairs with factor 1e30 are left unrotated (tests/test_transformer_cpp.cpp:137-158)
    assert np.allclose(gq[..., 16:32], q[..., 16:32], atol=1e-6)
    assert np.allclose(gq[..., 48:64], q[..., 48:64], atol=1e-6)


def test_rope_table_out_of_range_rows_untouched(hip, oracle):
    rng = np.random.default_rng(22)
    T, H, D = 6, 2, 32
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([0, 5, 99, -1, 7, 100], np.int32)
    cos, sin = oracle.rope_tables(D, np.arange(100, dtype=np.int32), 1e4)
    gq, _ = gpu_rope(q, pos, D, D, table=(cos, sin))
    for t in (3, 5):  # positions -1 and 100 fall outside the 100-row table
        assert bits_equal(gq[t], q[t])
    ok = [0, 1, 2, 4]
    wq = oracle_rope(oracle, q[ok], pos[ok], D, D, table=(cos, sin))
    assert bits_equal(gq[ok], wq)


def test_rope_relative_position_invariance(hip):
    """q.k depends only on the relative position (tests/test_transformer_cpp.cpp:
    227-257): the same q and k vectors at every token, k scored 5 tokens back."""
    rng = np.random.default_rng(23)
    T, D = 64, 128
    qv = rng.standard_normal(D).astype(np.float32)
    kv = rng.standard_normal(D).astype(np.float32)
    q = np.tile(qv, (T, 1, 1))
    k = np.tile(kv, (T, 1, 1))
    pos = np.arange(T, dtype=np.int32)
    for mode in (0, 1):
        gq, gk = gpu_rope(q, pos, D, D, k=k, theta=1e4, mode=mode)
        scores = (gq[5:, 0].astype(np.float64) * gk[:-5, 0]).sum(-1)
        assert np.abs(scores - scores[0]).max() < 1e-4


def test_rope_tables_device(hip, oracle):
    """Device rope_tables vs the oracle's (glibc sinf/cosf) at large positions."""
    for hd, nd, base in ((128, None, 5e5), (256, 64, 1e7), (64, None, 1e6)):
        pos = np.concatenate([np.arange(0, 32768, 7), [32767, 16383]]).astype(np.int32)
        n, inv = ops.rope_inv_freq(hd, nd, base)
        half = n // 2
        dc, ds = DA.empty((pos.size, half)), DA.empty((pos.size, half))
        ops.rope_tables(DA.from_numpy(pos), DA.from_numpy(inv), dc, ds)
        wc, ws = oracle.rope_tables(hd, pos, base, nd)
        assert rel_to_scale(dc.numpy(), wc) <= RTOL
        assert rel_to_scale(ds.numpy(), ws) <= RTOL


def test_rope_golden(hip):
    """The reference's own apply_rope outputs (NeoX, interleaved, partial 8)."""
    g = golden("ref_vectors.npz")
    x = g["apply_x"].reshape(6, 3, 32)
    pos = np.arange(6, dtype=np.int32)
    for key, mode, tab in (("apply_neox", 0, ("apply_cos", "apply_sin")),
                           ("apply_inter", 1, ("apply_cos", "apply_sin")),
                           ("apply_partial8", 0, ("apply_cos8", "apply_sin8"))):
        c, s = g[tab[0]], g[tab[1]]
        gq, _ = gpu_rope(x, pos, 32, 2 * c.shape[1], mode=mode, table=(c, s))
        assert bits_equal(gq.reshape(-1, 32), g[key]), key
