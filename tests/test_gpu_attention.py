"""GPU parity: the attention core and KV cache (aero_hip_attention /
aero_hip_kv_write / aero_hip_softmax_rows and the reference-compatible
aero_attention_tiled / aero_attention / aero_softmax*) against the oracle's
restatement of src/transformer.cpp:120-214, src/tensor.cpp:167-178 and
src/kv.cpp:13-46, and the reference's own outputs (tests/golden/ref_vectors.npz).

Attention and softmax: <= 1e-5 relative to the output's scale, the
reference's RTOL (tests/test_transformer_native.py:34-37,52-61); the GPU sums
in another order and uses its own exp. KV quantisation (integer codes and
scales): bit-exact.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, golden, rel_to_scale
from aero_amd import ops
from aero_amd import transformer_native as TN
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu


def gpu_attention(q, k, v, scale, qpos=None, kpos=None, window=0, kv_dt=0, ks=None, vs=None,
                  head_dim=None, value_dim=None):
    T, H, D = q.shape
    S, HK = k.shape[0], k.shape[1]
    D = head_dim or D
    DV = value_dim or v.shape[2]
    out = DA.empty((T, H, DV))
    dq = DA.from_numpy(np.ascontiguousarray(q, np.float32))
    dk, dv = DA.from_numpy(np.ascontiguousarray(k)), DA.from_numpy(np.ascontiguousarray(v))
    dqp = None if qpos is None else DA.from_numpy(np.asarray(qpos, np.int32))
    dkp = None if kpos is None else DA.from_numpy(np.asarray(kpos, np.int32))
    dks = None if ks is None else DA.from_numpy(np.asarray(ks, np.float32))
    dvs = None if vs is None else DA.from_numpy(np.asarray(vs, np.float32))
    ops.attention(dq, dk, dv, out, T, H, HK, D, DV, S, scale, qpos=dqp, kpos=dkp, window=window,
                  kv_dt=kv_dt, k_scale=dks, v_scale=dvs)
    return out.numpy()


def rand_qkv(rng, T, H, HK, D, DV, S):
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((S, HK, D)).astype(np.float32)
    v = rng.standard_normal((S, HK, DV)).astype(np.float32)
    return q, k, v


def test_attention_golden(hip):
    """The reference's own attention outputs: causal with positions (one query
    at a position below every key), a window, shuffled key positions."""
    g = golden("ref_vectors.npz")
    q, k, v, qpos = g["att_q"], g["att_k"], g["att_v"], g["att_qpos"]
    assert rel_to_scale(gpu_attention(q, k, v, 0.125, qpos=qpos), g["att_out"]) <= RTOL
    assert rel_to_scale(gpu_attention(q, k, v, 0.125, qpos=qpos, window=8),
                        g["att_out_win8"]) <= RTOL
    assert rel_to_scale(gpu_attention(q, k, v, 0.125, qpos=qpos, kpos=g["att_kpos"]),
                        g["att_out_kpos"]) <= RTOL
    # host ABI (engine/transformer_native.py shapes)
    assert rel_to_scale(TN.attention_tiled(q, k, v, 0.125, qpos=qpos), g["att_out"]) <= RTOL
    assert rel_to_scale(TN.softmax(g["softmax_x"]), g["softmax_y"]) <= RTOL


@pytest.mark.parametrize("T,H,HK,D,DV,S,window", [
    (1, 32, 8, 128, 128, 1, 0),        # decode, one key
    (1, 32, 8, 128, 128, 300, 0),      # decode, Llama-3-8B heads
    (1, 32, 8, 128, 128, 4096, 0),     # decode, 4k cache (key chunks + combine)
    (1, 64, 8, 128, 128, 2000, 0),     # 8 query heads per kv head
    (1, 14, 2, 64, 64, 777, 0),        # Qwen2-0.5B heads
    (1, 16, 2, 256, 256, 513, 0),      # head_dim 256 (Gemma-3 / Qwen3-next)
    (1, 32, 8, 128, 128, 1000, 64),    # sliding window
    (257, 8, 2, 128, 128, 257, 0),     # causal prefill
    (100, 6, 6, 80, 48, 130, 0),       # MHA, dims not a multiple of 16, value_dim < head_dim
    (33, 4, 1, 32, 32, 40, 7),         # MQA with a window
    (200, 8, 2, 128, 128, 300, 50),    # prefill after a cached prefix, with a window
    (3, 16, 4, 64, 64, 2500, 100),     # three tokens at once, head_dim 64, window
    (1, 8, 8, 128, 128, 5000, 0),      # MHA decode
    (100, 8, 4, 256, 256, 300, 0),     # head_dim 256 prefill after a cached prefix (matrix cores)
    (77, 16, 2, 256, 256, 77, 40),     # head_dim 256, 8 query heads a kv head, a window
    (1024, 8, 4, 256, 256, 1024, 0),   # Gemma-3-4B heads, 1024-token causal prefill
])
def test_attention_vs_oracle(hip, oracle, T, H, HK, D, DV, S, window):
    rng = np.random.default_rng(T * 7 + H + S + D + window)
    q, k, v = rand_qkv(rng, T, H, HK, D, DV, S)
    qpos = np.arange(S - T, S, dtype=np.int32)      # the last T positions (prefill / decode)
    scale = 1.0 / np.sqrt(D)
    print(f"attention T={T} H={H} HK={HK} D={D} DV={DV} S={S} window={window}", flush=True)
    got = gpu_attention(q, k, v, scale, qpos=qpos, window=window)
    want = oracle.attention_tiled(q, k, v, scale, qpos=qpos, window=window or None)
    assert rel_to_scale(got, want) <= RTOL


@pytest.mark.parametrize("D", [64, 256])
def test_attention_positions_and_masks(hip, oracle, D):
    """Arbitrary query / key positions (a shuffled cache), a query before every
    key (exact zeros), and the decode entry of the host ABI; head dims 64 and
    256 (both on the fp32 matrix-core kernel)."""
    rng = np.random.default_rng(5 + D)
    T, H, HK, S = 9, 8, 4, 70
    q, k, v = rand_qkv(rng, T, H, HK, D, D, S)
    qpos = np.array([-3, 0, 5, 69, 12, 40, 41, 100, 2], np.int32)
    kpos = rng.permutation(S).astype(np.int32)
    got = gpu_attention(q, k, v, 0.2, qpos=qpos, kpos=kpos)
    assert rel_to_scale(got, oracle.attention_tiled(q, k, v, 0.2, qpos=qpos, kpos=kpos)) <= RTOL
    assert not got[0].any()
    got_w = gpu_attention(q, k, v, 0.2, qpos=qpos, kpos=kpos, window=5)
    assert rel_to_scale(got_w, oracle.attention_tiled(q, k, v, 0.2, qpos=qpos, kpos=kpos,
                                                      window=5)) <= RTOL
    dq = rng.standard_normal((H, D)).astype(np.float32)
    assert rel_to_scale(TN.attention(dq, k, v, 0.2), oracle.attention(dq, k, v, 0.2)) <= RTOL


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_kv_write_bit_exact_and_ring(hip, oracle, dt):
    """Device quantisation of (token, head) vectors equals the reference's
    aero_kv_write_vec code for code and scale for scale, at ring positions
    (phys0 + t) % cap; includes a zero vector (scale 1) and a tiny one."""
    rng = np.random.default_rng(11 + dt)
    T, HK, D, cap, phys0 = 6, 3, 128, 8, 5
    x = (rng.standard_normal((T, HK, D)) * 4).astype(np.float32)
    x[1, 2] = 0.0
    x[3, 0] *= 1e-20
    vb = {0: 4 * D, 1: D, 2: D // 2}[dt]
    q = DA.empty(cap * HK * vb, np.uint8)
    sc = DA.empty(cap * HK)
    ops.kv_write(dt, DA.from_numpy(x), T, HK, D, q, sc, phys0, cap)
    qh = q.numpy().reshape(cap, HK, vb)
    sh = sc.numpy().reshape(cap, HK)
    for t in range(T):
        p = (phys0 + t) % cap
        for h in range(HK):
            want_q, want_s = oracle.kv_write_vec(dt, x[t, h])
            assert np.array_equal(qh[p, h], want_q), (t, h)
            if dt:
                assert np.float32(sh[p, h]) == np.float32(want_s), (t, h)
    if dt:  # host ABI, one vector
        from aero_amd import _lib
        import ctypes
        qb = np.zeros(vb, np.uint8)
        s1 = np.zeros(1, np.float32)
        assert _lib.lib().aero_kv_write_vec(dt, x[0, 0].ctypes.data_as(
            ctypes.POINTER(ctypes.c_float)), D, qb.ctypes.data, s1.ctypes.data_as(
            ctypes.POINTER(ctypes.c_float))) == 1
        wq, ws = oracle.kv_write_vec(dt, x[0, 0])
        assert np.array_equal(qb, wq) and np.float32(s1[0]) == np.float32(ws)


@pytest.mark.parametrize("dt,T,H,HK,D,S", [(1, 3, 32, 8, 128, 1500), (2, 3, 32, 8, 128, 1500),
                                           (1, 40, 14, 2, 64, 700), (2, 1, 14, 2, 64, 3000),
                                           # several 32-key steps a wave (4 a chunk of 512),
                                           # a partial last chunk
                                           (1, 64, 32, 8, 128, 2048), (2, 64, 32, 8, 128, 2048),
                                           (1, 1, 32, 8, 128, 32768), (2, 1, 32, 8, 64, 20000),
                                           # head_dim 256 (the fp32 matrix-core kernel
                                           # reading the codes): decode and prefill
                                           (1, 1, 8, 4, 256, 3000), (2, 1, 8, 4, 256, 3000),
                                           (1, 70, 16, 2, 256, 300), (2, 70, 16, 2, 256, 300)])
def test_attention_over_quantised_cache(hip, oracle, dt, T, H, HK, D, S):
    """Attention reading an int8 / int4 cache (the fp16 matrix-core kernel at
    head dims 64 and 128) equals the oracle's attention over the cache read
    back with the reference's aero_kv_read_vec."""
    rng = np.random.default_rng(23 + dt + T)
    print(f"quantised-cache attention dt={dt} T={T} H={H}/{HK} D={D} S={S}", flush=True)
    q, k, v = rand_qkv(rng, T, H, HK, D, D, S)
    vb = D if dt == 1 else D // 2
    kq, vq = DA.empty(S * HK * vb, np.uint8), DA.empty(S * HK * vb, np.uint8)
    ks, vs = DA.empty(S * HK), DA.empty(S * HK)
    ops.kv_write(dt, DA.from_numpy(k), S, HK, D, kq, ks, 0, S)
    ops.kv_write(dt, DA.from_numpy(v), S, HK, D, vq, vs, 0, S)
    kqh, vqh = kq.numpy().reshape(S * HK, vb), vq.numpy().reshape(S * HK, vb)
    ksh, vsh = ks.numpy(), vs.numpy()
    kd = np.stack([oracle.kv_read_vec(dt, kqh[i], ksh[i], D) for i in range(S * HK)])
    vd = np.stack([oracle.kv_read_vec(dt, vqh[i], vsh[i], D) for i in range(S * HK)])
    kd, vd = kd.reshape(S, HK, D), vd.reshape(S, HK, D)
    qpos = np.arange(S - T, S, dtype=np.int32)
    out = DA.empty((T, H, D))
    ops.attention(DA.from_numpy(q), kq, vq, out, T, H, HK, D, D, S, 0.09,
                  qpos=DA.from_numpy(qpos), kv_dt=dt, k_scale=ks, v_scale=vs)
    want = oracle.attention_tiled(q, kd, vd, 0.09, qpos=qpos)
    assert rel_to_scale(out.numpy(), want) <= RTOL


@pytest.mark.parametrize("dt,D,H,HK,S", [(1, 64, 8, 2, 700), (2, 64, 8, 2, 700),
                                          (1, 128, 32, 8, 6000), (2, 128, 32, 8, 6000),
                                          (1, 256, 8, 4, 700), (2, 256, 8, 4, 700)])
def test_quantised_cache_positions_and_masks(hip, oracle, dt, D, H, HK, S):
    """The integer-cache kernels (fp16 matrix steps at head dims 64 and 128,
    the fp32 matrix-core kernel reading the codes at 256) under arbitrary
    positions: a shuffled cache (700 keys: one 32-key step a wave; 6000 keys:
    chunks of 384, three steps a wave), a query before every key (exact
    zeros), positions past the cache, then the same with a window of 37."""
    rng = np.random.default_rng(11 * dt + D)
    T = 9
    print(f"quantised-cache positions dt={dt} D={D} S={S}", flush=True)
    q, k, v = rand_qkv(rng, T, H, HK, D, D, S)
    vb = D if dt == 1 else D // 2
    kq, vq = DA.empty(S * HK * vb, np.uint8), DA.empty(S * HK * vb, np.uint8)
    ks, vs = DA.empty(S * HK), DA.empty(S * HK)
    ops.kv_write(dt, DA.from_numpy(k), S, HK, D, kq, ks, 0, S)
    ops.kv_write(dt, DA.from_numpy(v), S, HK, D, vq, vs, 0, S)
    kqh, vqh = kq.numpy().reshape(S * HK, vb), vq.numpy().reshape(S * HK, vb)
    ksh, vsh = ks.numpy(), vs.numpy()
    kd = np.stack([oracle.kv_read_vec(dt, kqh[i], ksh[i], D) for i in range(S * HK)])
    vd = np.stack([oracle.kv_read_vec(dt, vqh[i], vsh[i], D) for i in range(S * HK)])
    kd, vd = kd.reshape(S, HK, D), vd.reshape(S, HK, D)
    qpos = np.array([-3, 0, 5, S - 1, 120, 400, 401, S + 300, 2], np.int32)
    kpos = rng.permutation(S).astype(np.int32)
    for window in (0, 37):
        out = DA.empty((T, H, D))
        ops.attention(DA.from_numpy(q), kq, vq, out, T, H, HK, D, D, S, 0.11,
                      qpos=DA.from_numpy(qpos), kpos=DA.from_numpy(kpos), window=window,
                      kv_dt=dt, k_scale=ks, v_scale=vs)
        want = oracle.attention_tiled(q, kd, vd, 0.11, qpos=qpos, kpos=kpos,
                                      window=window or None)
        got = out.numpy()
        assert rel_to_scale(got, want) <= RTOL, window
        assert not got[0].any()


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("case", ["late_jump", "tiny_block"])
@pytest.mark.parametrize("one_chunk", [False, True])
def test_quantised_cache_scale_ranges(hip, oracle, dt, case, one_chunk):
    """Value vectors in blocks of 1e-30, 1e24, 1, 1e-20 and 3 along the cache
    (value scales 2^-100 .. 2^80), keys of the 1e24 block (and, for
    tiny_block, of every block but 1e-20) pointing away from the queries so
    their weights vanish, and a late key whose score jumps far above the
    running max (late_jump) or an output carried by the 1e-20 block alone
    (tiny_block). The integer-cache kernel keeps its value sums in units of a
    per-step power of two and its probabilities against a reference max that
    moves only on large changes; with one chunk every wave walks ~23 steps in
    one pass and meets each change. Against the oracle's attention over the
    read-back cache."""
    from aero_amd.device import tune_set
    rng = np.random.default_rng(91 + dt + 2 * one_chunk)
    T, H, HK, D, S = 1, 8, 2, 128, 3000
    q, k, v = rand_qkv(rng, T, H, HK, D, D, S)
    mags = np.ones(S, np.float32)
    mags[0:400], mags[400:800], mags[1600:2400], mags[2400:] = 1e-30, 1e24, 1e-20, 3.0
    v = (v * mags[:, None, None]).astype(np.float32)
    qdir = q[0].reshape(HK, H // HK, D).sum(1)
    qdir = qdir / np.linalg.norm(qdir, axis=-1, keepdims=True)
    away = list(range(400, 800)) if case == "late_jump" else \
        list(range(400, 1600)) + list(range(2400, S))
    k[away] = -qdir[None] * 4000.0
    if case == "late_jump":
        k[2990] = qdir * 30.0
    else:
        k[1600:2400] = k[1600:2400] * 0.2 + qdir[None] * 10.0
    vb = D if dt == 1 else D // 2
    kq, vq = DA.empty(S * HK * vb, np.uint8), DA.empty(S * HK * vb, np.uint8)
    ks, vs = DA.empty(S * HK), DA.empty(S * HK)
    ops.kv_write(dt, DA.from_numpy(k.astype(np.float32)), S, HK, D, kq, ks, 0, S)
    ops.kv_write(dt, DA.from_numpy(v), S, HK, D, vq, vs, 0, S)
    kqh, vqh = kq.numpy().reshape(S * HK, vb), vq.numpy().reshape(S * HK, vb)
    ksh, vsh = ks.numpy(), vs.numpy()
    kd = np.stack([oracle.kv_read_vec(dt, kqh[i], ksh[i], D) for i in range(S * HK)])
    vd = np.stack([oracle.kv_read_vec(dt, vqh[i], vsh[i], D) for i in range(S * HK)])
    kd, vd = kd.reshape(S, HK, D), vd.reshape(S, HK, D)
    qpos = np.array([S - 1], np.int32)
    want = oracle.attention_tiled(q, kd, vd, 0.09, qpos=qpos)
    scale = np.abs(want).max()
    if case == "tiny_block":
        assert 1e-24 < scale < 1e-16   # carried by the 1e-20 block
    else:
        assert 0.5 < scale < 20.0      # carried by the late key (3.0 block)
    print(f"scale ranges dt={dt} {case} one_chunk={one_chunk}", flush=True)
    out = DA.empty((T, H, D))
    if one_chunk:
        tune_set("attn_wgs", 1)
    try:
        ops.attention(DA.from_numpy(q), kq, vq, out, T, H, HK, D, D, S, 0.09,
                      qpos=DA.from_numpy(qpos), kv_dt=dt, k_scale=ks, v_scale=vs)
        got = out.numpy()
    finally:
        if one_chunk:
            tune_set("attn_wgs", None)
    assert np.isfinite(got).all()
    assert rel_to_scale(got, want) <= RTOL


@pytest.mark.parametrize("combine4", [1, 0])
@pytest.mark.parametrize("dt,H,HK,D,DV,S", [(0, 32, 8, 128, 128, 4096), (0, 16, 2, 256, 256, 3000),
                                             (0, 14, 2, 64, 48, 2500), (1, 8, 2, 42, 42, 3000),
                                             (1, 32, 8, 128, 128, 9000)])
def test_chunk_merge_kernels(hip, oracle, combine4, dt, H, HK, D, DV, S):
    """Decode over many key chunks: the chunk merge with float4 lanes (value
    widths of a multiple of 4) and the scalar one (attn_combine4=0, and the
    42-wide int8 value rows, which always take it) both equal the oracle."""
    from aero_amd.device import tune_set
    rng = np.random.default_rng(31 + D + S)
    q, k, v = rand_qkv(rng, 1, H, HK, D, DV, S)
    qpos = np.array([S - 1], np.int32)
    print(f"chunk merge combine4={combine4} dt={dt} H={H}/{HK} D={D} DV={DV} S={S}", flush=True)
    if dt == 0:
        kd, vd, args = k, v, {}
    else:
        kq, vq = DA.empty(S * HK * D, np.uint8), DA.empty(S * HK * DV, np.uint8)
        ks, vs = DA.empty(S * HK), DA.empty(S * HK)
        ops.kv_write(dt, DA.from_numpy(k), S, HK, D, kq, ks, 0, S)
        ops.kv_write(dt, DA.from_numpy(v), S, HK, DV, vq, vs, 0, S)
        kqh, vqh = kq.numpy().reshape(S * HK, D), vq.numpy().reshape(S * HK, DV)
        ksh, vsh = ks.numpy(), vs.numpy()
        kd = np.stack([oracle.kv_read_vec(dt, kqh[i], ksh[i], D)
                       for i in range(S * HK)]).reshape(S, HK, D)
        vd = np.stack([oracle.kv_read_vec(dt, vqh[i], vsh[i], DV)
                       for i in range(S * HK)]).reshape(S, HK, DV)
        args = dict(kv_dt=dt, k_scale=ks, v_scale=vs)
    out = DA.empty((1, H, DV))
    dk = DA.from_numpy(k) if dt == 0 else kq
    dv = DA.from_numpy(v) if dt == 0 else vq
    tune_set("attn_combine4", combine4)
    try:
        ops.attention(DA.from_numpy(q), dk, dv, out, 1, H, HK, D, DV, S, 0.11,
                      qpos=DA.from_numpy(qpos), **args)
        got = out.numpy()
    finally:
        tune_set("attn_combine4", None)
    want = oracle.attention_tiled(q, kd, vd, 0.11, qpos=qpos)
    assert rel_to_scale(got, want) <= RTOL


def test_softmax_rows(hip, oracle):
    """Rows of 1..100k values, large and tiny ranges; the flat-vector host ABI."""
    rng = np.random.default_rng(31)
    for rows, cols, s in ((1, 1, 1.0), (3, 7, 50.0), (64, 4096, 3.0), (2, 100000, 10.0)):
        x = (rng.standard_normal((rows, cols)) * s).astype(np.float32)
        dx, dy = DA.from_numpy(x), DA.empty((rows, cols))
        ops.softmax_rows(dx, dy, rows, cols)
        assert rel_to_scale(dy.numpy(), oracle.softmax(x)) <= RTOL
    from aero_amd import tensor_native
    x = (rng.standard_normal(1000) * 5).astype(np.float32)
    xc = x.copy()
    y = tensor_native.softmax(xc)
    # in place on a contiguous float32 input, as engine/tensor_native.py:153-160
    assert np.shares_memory(y, xc)
    assert rel_to_scale(y, oracle.softmax(x)) <= RTOL


def test_attention_decode_full_size(hip, oracle):
    """Llama-3-8B decode at a 16k-token cache (H=32, HK=8, D=128): the key split
    into chunks and their combine against the oracle; and the 512-token causal
    prefill of the same heads."""
    rng = np.random.default_rng(37)
    q, k, v = rand_qkv(rng, 1, 32, 8, 128, 128, 16384)
    got = gpu_attention(q, k, v, 1 / np.sqrt(128), qpos=[16383])
    assert rel_to_scale(got, oracle.attention_tiled(q, k, v, 1 / np.sqrt(128),
                                                    qpos=[16383])) <= RTOL
    q, k, v = rand_qkv(rng, 512, 32, 8, 128, 128, 512)
    got = gpu_attention(q, k, v, 1 / np.sqrt(128))
    assert rel_to_scale(got, oracle.attention_tiled(q, k, v, 1 / np.sqrt(128))) <= RTOL


def _random_attention_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dt = int(rng.integers(0, 3))
        D = int(rng.choice([64, 128]))
        HK = int(rng.choice([1, 2, 4, 8]))
        H = HK * int(rng.choice([1, 2, 4, 7, 8]))
        T = int(rng.integers(1, 71))
        S = int(rng.integers(T, 3001))
        window = int(rng.choice([0, 0, int(rng.integers(1, S + 1))]))
        cases.append((i, dt, T, H, HK, D, S, window))
    return cases


@pytest.mark.parametrize("i,dt,T,H,HK,D,S,window", _random_attention_cases(24, 2026))
def test_attention_random_shapes(hip, oracle, i, dt, T, H, HK, D, S, window):
    """Seeded random shapes over every cache type and both matrix-core kernels:
    1-70 queries at the last positions of 1-3000 keys, 1-8 query heads a kv
    head, head dims 64 / 128, with and without a window."""
    rng = np.random.default_rng(100 + i)
    print(f"random attention {i}: dt={dt} T={T} H={H}/{HK} D={D} S={S} window={window}",
          flush=True)
    q, k, v = rand_qkv(rng, T, H, HK, D, D, S)
    qpos = np.arange(S - T, S, dtype=np.int32)
    scale = 1.0 / np.sqrt(D)
    if dt == 0:
        got = gpu_attention(q, k, v, scale, qpos=qpos, window=window)
        want = oracle.attention_tiled(q, k, v, scale, qpos=qpos, window=window or None)
    else:
        vb = D if dt == 1 else D // 2
        kq, vq = DA.empty(S * HK * vb, np.uint8), DA.empty(S * HK * vb, np.uint8)
        ks, vs = DA.empty(S * HK), DA.empty(S * HK)
        ops.kv_write(dt, DA.from_numpy(k), S, HK, D, kq, ks, 0, S)
        ops.kv_write(dt, DA.from_numpy(v), S, HK, D, vq, vs, 0, S)
        kqh, vqh = kq.numpy().reshape(S * HK, vb), vq.numpy().reshape(S * HK, vb)
        ksh, vsh = ks.numpy(), vs.numpy()
        kd = np.stack([oracle.kv_read_vec(dt, kqh[j], ksh[j], D)
                       for j in range(S * HK)]).reshape(S, HK, D)
        vd = np.stack([oracle.kv_read_vec(dt, vqh[j], vsh[j], D)
                       for j in range(S * HK)]).reshape(S, HK, D)
        out = DA.empty((T, H, D))
        ops.attention(DA.from_numpy(q), kq, vq, out, T, H, HK, D, D, S, scale,
                      qpos=DA.from_numpy(qpos), window=window, kv_dt=dt, k_scale=ks,
                      v_scale=vs)
        got = out.numpy()
        want = oracle.attention_tiled(q, kd, vd, scale, qpos=qpos, window=window or None)
    assert rel_to_scale(got, want) <= RTOL
