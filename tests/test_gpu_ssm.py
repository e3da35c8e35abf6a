"""GPU parity: the gated DeltaNet scan and causal conv (aero_hip_ssm_scan,
aero_hip_ssm_conv and the reference-compatible aero_ssm_* host ABI) against
the oracle's restatement of src/ssm.cpp:17-210 and the reference's own outputs
(tests/golden/ref_vectors.npz).

Scan outputs and states: <= 1e-5 relative to their scale (the reference's
TOL, tests/test_ssm_native.py:36-37); the GPU sums in another order and uses
its own exp / log1p / sqrt. Conv: bit-exact (taps added in the reference's
order, separate multiplies and adds).
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, golden, rel_to_scale
from aero_amd import _lib
from aero_amd import native_ssm as NS
from aero_amd import ops
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu


def inputs(rng, T, n_k, n_v, d):
    q = rng.standard_normal((T, n_k, d)).astype(np.float32)
    k = rng.standard_normal((T, n_k, d)).astype(np.float32)
    v = rng.standard_normal((T, n_v, d)).astype(np.float32)
    alpha = rng.standard_normal((T, n_v)).astype(np.float32)
    beta = rng.standard_normal((T, n_v)).astype(np.float32)
    a_log = (-np.abs(rng.standard_normal(n_v)) * 0.5).astype(np.float32)
    dt_bias = rng.standard_normal(n_v).astype(np.float32)
    state = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
    return q, k, v, alpha, beta, a_log, dt_bias, state


def gpu_scan(q, k, v, alpha, beta, a_log, dt_bias, state, scale, eps=1e-6, dstate=None):
    T, n_k, d = q.shape
    n_v = v.shape[1]
    if dstate is None:
        dstate = DA.from_numpy(state)
    outs = DA.empty((T, n_v, d))
    ops.ssm_scan(DA.from_numpy(q), DA.from_numpy(k), DA.from_numpy(v), DA.from_numpy(alpha),
                 DA.from_numpy(beta), DA.from_numpy(a_log), DA.from_numpy(dt_bias), dstate,
                 outs, T, n_k, n_v, d, scale, eps)
    return outs.numpy(), dstate


def test_scan_and_conv_golden(hip):
    """The reference's own scan (6 tokens, 2 k-heads, 4 v-heads, d 32 is below
    the device kernel's widths: checked through the 64-wide zero-padded
    equivalent) and conv outputs."""
    g = golden("ref_vectors.npz")
    # zero-pad d 32 -> 64: padded q/k elements change no norm, padded v
    # columns stay zero, the first 32 columns are the reference's
    pad = lambda a, ax: np.concatenate([a, np.zeros_like(a)], axis=ax)
    st = np.zeros((4, 64, 64), np.float32)
    st[:, :32, :32] = g["ssm_state"]
    out, dst = gpu_scan(pad(g["ssm_q"], 2), pad(g["ssm_k"], 2), pad(g["ssm_v"], 2),
                        g["ssm_alpha"], g["ssm_beta"], g["ssm_a_log"], g["ssm_dt_bias"], st,
                        0.125)
    assert rel_to_scale(out[:, :, :32], g["ssm_out"]) <= RTOL
    assert not out[:, :, 32:].any()
    assert rel_to_scale(dst.numpy()[:, :32, :32], g["ssm_state_out"]) <= RTOL
    o1, t1, l1 = NS.conv(g["conv_x"][:2], g["conv_w"], None, 0)
    o2, t2, l2 = NS.conv(g["conv_x"][2:], g["conv_w"], t1, l1)
    assert bits_equal(np.concatenate([o1, o2]), g["conv_out"]) and bits_equal(t2, g["conv_tail"])


@pytest.mark.parametrize("T,n_k,n_v,d", [
    (1, 16, 32, 128),      # Qwen3-Next decode: 16 key heads, 32 value heads, d 128
    (64, 16, 32, 128),     # a 64-token prefill chunk at the same heads
    (300, 2, 4, 64),       # d 64, v-heads in two groups of a key head
    (20, 1, 2, 256),       # d 256
    (33, 3, 3, 128),       # one value head per key head
])
def test_scan_vs_oracle(hip, oracle, T, n_k, n_v, d):
    rng = np.random.default_rng(T + 7 * n_v + d)
    args = inputs(rng, T, n_k, n_v, d)
    print(f"ssm scan T={T} n_k={n_k} n_v={n_v} d={d}", flush=True)
    scale = 1.0 / np.sqrt(d)
    out, dst = gpu_scan(*args, scale)
    want, wst = oracle.ssm_scan(*args, scale)
    assert rel_to_scale(out, want) <= RTOL
    assert rel_to_scale(dst.numpy(), wst) <= RTOL


@pytest.mark.parametrize("T,n_k,n_v,d", [
    (128, 16, 32, 128),    # two whole 64-token chunks at Qwen3-Next's heads
    (300, 2, 4, 128),      # a partial last chunk (44 tokens)
    (129, 1, 2, 128),      # a last chunk of one token
    (256, 4, 4, 128),      # one value head a key head
    (1000, 3, 6, 128),     # 16 chunks, two value heads a key head
    # head dims 64 and 256: the lean state pass
    (128, 4, 8, 64),
    (300, 2, 4, 64),
    (129, 1, 2, 64),
    (1000, 3, 6, 64),
    (128, 2, 4, 256),
    (300, 1, 2, 256),
    (129, 2, 2, 256),
    (700, 1, 3, 256),
])
def test_chunked_scan_vs_oracle(hip, oracle, T, n_k, n_v, d):
    """Scans of 128 or more tokens take the chunked (WY) form: chunk pre-pass +
    state pass on the matrix cores; same tolerance."""
    rng = np.random.default_rng(T + n_k + d)
    args = inputs(rng, T, n_k, n_v, d)
    print(f"chunked ssm scan T={T} n_k={n_k} n_v={n_v} d={d}", flush=True)
    scale = d ** -0.5
    out, dst = gpu_scan(*args, scale)
    want, wst = oracle.ssm_scan(*args, scale)
    assert rel_to_scale(out, want) <= RTOL
    assert rel_to_scale(dst.numpy(), wst) <= RTOL


@pytest.mark.parametrize("d", [128, 64, 256])
def test_chunked_scan_strong_decay_and_chain(hip, oracle, d):
    """Decays near zero (a_log -30: exp(L) underflows inside a chunk) and near
    one, gates near 0 and 1; two chunked calls of 200 tokens carrying the
    state equal one of 400 and the oracle."""
    rng = np.random.default_rng(77 + d)
    print(f"chunked ssm scan chain d={d}", flush=True)
    q, k, v, al, bt, a_log, dt, st = inputs(rng, 400, 2, 4, d)
    a_log = np.array([-30.0, -1e-4, -0.5, -3.0], np.float32)
    bt[:, 0] = 20.0                                    # gate 1
    bt[:, 1] = -20.0                                   # gate ~0
    scale = d ** -0.5
    whole, wst = gpu_scan(q, k, v, al, bt, a_log, dt, st, scale)
    want, ost = oracle.ssm_scan(q, k, v, al, bt, a_log, dt, st, scale)
    assert rel_to_scale(whole, want) <= RTOL and rel_to_scale(wst.numpy(), ost) <= RTOL
    dst = DA.from_numpy(st)
    a, _ = gpu_scan(q[:200], k[:200], v[:200], al[:200], bt[:200], a_log, dt, None, scale,
                    dstate=dst)
    b, _ = gpu_scan(q[200:], k[200:], v[200:], al[200:], bt[200:], a_log, dt, None, scale,
                    dstate=dst)
    assert rel_to_scale(np.concatenate([a, b]), want) <= RTOL
    assert rel_to_scale(dst.numpy(), ost) <= RTOL
    assert np.isfinite(whole).all()


def test_scan_decode_chain_and_host_abi(hip, oracle):
    """Three one-token calls carrying the state equal one three-token call
    (the state is updated in place on the device); the host ABI's scan and
    delta_step equal the oracle and leave the caller's state untouched."""
    rng = np.random.default_rng(61)
    q, k, v, al, bt, a_log, dt, st = inputs(rng, 3, 16, 32, 128)
    scale = 1.0 / np.sqrt(128)
    dst = DA.from_numpy(st)
    steps = [gpu_scan(q[t:t + 1], k[t:t + 1], v[t:t + 1], al[t:t + 1], bt[t:t + 1], a_log, dt,
                      None, scale, dstate=dst)[0] for t in range(3)]
    whole, wst = gpu_scan(q, k, v, al, bt, a_log, dt, st, scale)
    assert rel_to_scale(np.concatenate(steps), whole) <= RTOL
    assert rel_to_scale(dst.numpy(), wst.numpy()) <= RTOL
    st0 = st.copy()
    outs, nst = NS.scan(q, k, v, al, bt, a_log, dt, st, scale)
    want, wst2 = oracle.ssm_scan(q, k, v, al, bt, a_log, dt, st, scale)
    assert rel_to_scale(outs, want) <= RTOL and rel_to_scale(nst, wst2) <= RTOL
    assert bits_equal(st, st0)
    qe, ke = np.tile(q[0], (2, 1)), np.tile(k[0], (2, 1))     # tiled to the 32 v-heads
    o1, s1 = NS.delta_step(qe, ke, v[0], al[0], bt[0], a_log, dt, st, scale)
    w1, ws1 = oracle.ssm_delta_step(qe, ke, v[0], al[0], bt[0], a_log, dt, st, scale)
    assert rel_to_scale(o1, w1) <= RTOL and rel_to_scale(s1, ws1) <= RTOL
    xs = np.linspace(-30, 30, 121).astype(np.float32)
    assert rel_to_scale(NS.softplus(xs), oracle.ssm_softplus(xs)) <= 1e-6


def test_scan_full_prefill_by_segments(hip, oracle):
    """Qwen3-Next's 4096-token prefill (16 key heads, 32 value heads, d 128):
    one call equals two 2048-token calls carrying the state, and the last 64
    tokens equal the oracle's scan started from the GPU's state at token 4032."""
    rng = np.random.default_rng(67)
    T = 4096
    q, k, v, al, bt, a_log, dt, st = inputs(rng, T, 16, 32, 128)
    scale = 1.0 / np.sqrt(128)
    whole, wst = gpu_scan(q, k, v, al, bt, a_log, dt, st, scale)
    dst = DA.from_numpy(st)
    a, _ = gpu_scan(q[:2048], k[:2048], v[:2048], al[:2048], bt[:2048], a_log, dt, None,
                    scale, dstate=dst)
    b, _ = gpu_scan(q[2048:4032], k[2048:4032], v[2048:4032], al[2048:4032], bt[2048:4032],
                    a_log, dt, None, scale, dstate=dst)
    mid = dst.numpy()
    c, _ = gpu_scan(q[4032:], k[4032:], v[4032:], al[4032:], bt[4032:], a_log, dt, None,
                    scale, dstate=dst)
    assert rel_to_scale(np.concatenate([a, b, c]), whole) <= RTOL
    assert rel_to_scale(dst.numpy(), wst.numpy()) <= RTOL
    want, wend = oracle.ssm_scan(q[4032:], k[4032:], v[4032:], al[4032:], bt[4032:], a_log, dt,
                                 mid, scale)
    assert rel_to_scale(c, want) <= RTOL and rel_to_scale(dst.numpy(), wend) <= RTOL
    assert np.isfinite(whole).all() and np.abs(wst.numpy()).max() < 1e3


@pytest.mark.parametrize("T,C,K,chunks", [(7, 10, 4, [2, 5]), (1, 8192, 4, [1, 1, 1, 1]),
                                          (300, 1000, 4, [150, 150]), (5, 33, 1, [5]),
                                          (9, 64, 6, [1, 2, 6]), (1000, 8192, 4, [500, 500])])
def test_conv_bit_exact(hip, oracle, T, C, K, chunks):
    """Against the oracle chunk by chunk (tails shorter than kernel - 1 while
    the history fills), through the device op with the tail updated in place
    and through the host ABI."""
    rng = np.random.default_rng(T + C + K)
    x = rng.standard_normal((sum(chunks), C)).astype(np.float32)
    w = rng.standard_normal((C, K)).astype(np.float32)
    dw = DA.from_numpy(w)
    dtail = DA.empty(max(K - 1, 1) * C)
    tl = 0
    otail, otl = None, 0
    htail, htl = None, 0
    pos = 0
    for n in chunks:
        xc = x[pos:pos + n]
        want, otail, otl = oracle.ssm_conv(xc, w, otail, otl)
        dout = DA.empty((n, C))
        tl = ops.ssm_conv(DA.from_numpy(xc), dw, dtail if tl else None, tl,
                          dtail if K > 1 else None, dout, n, C, K)
        assert tl == otl
        assert bits_equal(dout.numpy(), want)
        if tl:
            assert bits_equal(dtail.numpy()[:tl * C].reshape(tl, C), otail[:tl])
        hout, htail, htl = NS.conv(xc, w, htail, htl)
        assert bits_equal(hout, want) and htl == otl
        pos += n


def test_workspace_grows_and_is_reused(hip, oracle):
    """One workspace serves every size: a 300-token chunked scan, then 40
    tokens (per-token loop, smaller workspace), then 129 (chunked again);
    each equals the oracle and a single buffer of the largest size is kept."""
    rng = np.random.default_rng(91)
    scale = 128 ** -0.5
    for T in (300, 40, 129):
        args = inputs(rng, T, 2, 4, 128)
        out, dst = gpu_scan(*args, scale)
        want, wst = oracle.ssm_scan(*args, scale)
        assert rel_to_scale(out, want) <= RTOL and rel_to_scale(dst.numpy(), wst) <= RTOL
    assert ops._ssm_ws.buf.nbytes >= _lib.lib().aero_hip_ssm_workspace(300, 2, 4, 128)


@pytest.mark.parametrize("T", [5, 40, 200])
def test_scan_strided_equals_contiguous(hip, T):
    """q, k, v as slices of packed rows (with 8 floats of padding a row) give
    the contiguous scan's outputs and state bit for bit, on the fused (5
    tokens), per-token (40) and chunked (200) paths."""
    rng = np.random.default_rng(T)
    n_k, n_v, d = 2, 4, 128
    q, k, v, al, bt, a_log, dt, st = inputs(rng, T, n_k, n_v, d)
    W_ = 2 * n_k * d + n_v * d + 8
    packed = np.zeros((T, W_), np.float32)
    packed[:, :n_k * d] = q.reshape(T, -1)
    packed[:, n_k * d:2 * n_k * d] = k.reshape(T, -1)
    packed[:, 2 * n_k * d:2 * n_k * d + n_v * d] = v.reshape(T, -1)
    print(f"strided scan T={T}", flush=True)
    want, wst = gpu_scan(q, k, v, al, bt, a_log, dt, st, d ** -0.5)
    dp, sdev, outs = DA.from_numpy(packed), DA.from_numpy(st), DA.empty((T, n_v, d))
    ops.ssm_scan(dp, dp, dp, DA.from_numpy(al), DA.from_numpy(bt), DA.from_numpy(a_log),
                 DA.from_numpy(dt), sdev, outs, T, n_k, n_v, d, d ** -0.5,
                 strides=(W_, W_, W_), q_off=0, k_off=n_k * d, v_off=2 * n_k * d)
    assert bits_equal(outs.numpy(), want) and bits_equal(sdev.numpy(), wst.numpy())


def test_scan_strided_refusals(hip):
    rng = np.random.default_rng(3)
    T, n_k, n_v, d = 4, 1, 2, 64
    q, k, v, al, bt, a_log, dt, st = inputs(rng, T, n_k, n_v, d)
    L = _lib.lib()
    dq, dv, da = DA.from_numpy(q), DA.from_numpy(v), DA.from_numpy(al)
    ds, do = DA.from_numpy(st), DA.empty((T, n_v, d))
    ws = DA.empty((L.aero_hip_ssm_workspace(T, n_k, n_v, d) // 4 + 64,))
    for qs, vs in ((n_k * d - 4, n_v * d), (n_k * d + 2, n_v * d), (n_k * d, n_v * d - 64)):
        assert L.aero_hip_ssm_scan_strided(dq.ptr, qs, dq.ptr, qs, dv.ptr, vs, da.ptr, da.ptr,
                                           da.ptr, da.ptr, ds.ptr, T, n_k, n_v, d, 0.1, 1e-6,
                                           do.ptr, ws.ptr, ws.nbytes, None) == 0
        assert "strides" in _lib.last_error()


@pytest.mark.parametrize("T,C,K,chunks", [(40, 1000, 4, [1, 2, 37]), (300, 1024, 4, [3, 297]),
                                          (9, 64, 6, [4, 5])])
def test_conv_silu(hip, oracle, T, C, K, chunks):
    """The conv with silu in its store equals the oracle's conv then
    x / (1 + exp(-x)) (1e-6 of scale: the GPU's exp), and its history
    (written by the one-block kernel below 33 tokens) is the plain conv's, bit
    for bit, over chunks carrying it."""
    rng = np.random.default_rng(T + C)
    x = rng.standard_normal((T, C)).astype(np.float32)
    w = rng.standard_normal((C, K)).astype(np.float32)
    tail = DA.empty((K - 1, C))
    tl, otail, otl, a = 0, np.zeros((K - 1, C), np.float32), 0, 0
    for n in chunks:
        print(f"conv silu chunk {a}:{a + n} of C={C} K={K}", flush=True)
        out = DA.empty((n, C))
        tl = ops.ssm_conv(DA.from_numpy(x[a:a + n]), DA.from_numpy(w), tail, tl, tail, out, n, C,
                          K, silu=True)
        want, otail, otl = oracle.ssm_conv(x[a:a + n], w, otail, otl)
        want = want / (np.float32(1) + np.exp(-want))
        assert rel_to_scale(out.numpy(), want) <= 1e-6
        assert tl == otl and bits_equal(tail.numpy()[:tl], otail[:otl])
        a += n
