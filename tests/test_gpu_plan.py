"""GPU: a recorded plan replays exactly the kernels its ops would have
launched (bit-identical results), any number of times, with per-kernel
timing events; recording launches nothing."""
import numpy as np
import pytest

from conftest import bits_equal
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA, Event, Plan, Stream

pytestmark = pytest.mark.gpu


def _inputs(seed):
    s = W.SHAPES["llama3_8b_prefill"]
    rng = np.random.default_rng(seed)
    R = 64
    d = {
        "x": rng.standard_normal((R, s.hidden), dtype=np.float32),
        "w": (1 + 0.1 * rng.standard_normal(s.hidden)).astype(np.float32),
        "q": rng.standard_normal((R, s.hq, s.head_dim), dtype=np.float32),
        "k": rng.standard_normal((R, s.hk, s.head_dim), dtype=np.float32),
        "g": rng.standard_normal((R, 1000), dtype=np.float32),
        "u": rng.standard_normal((R, 1000), dtype=np.float32),
        "pos": np.arange(R, dtype=np.int32),
    }
    e = W.embed_inputs(s, vocab=300, rows=R)
    return s, d, e


def _record_or_run(s, dev, e, inv):
    R = 64
    ops.embed_gather(e["type"], dev["tab"], e["vocab"], s.hidden, dev["ids"], dev["emb"])
    ops.rmsnorm(dev["x"], dev["w"], dev["h"], R, s.hidden, s.eps)
    ops.qk_norm_rope(dev["q"], s.hq, R, s.head_dim, s.n_rot, k=dev["k"], n_k_heads=s.hk,
                     pos=dev["pos"], inv_freq=inv)
    ops.act_mul("silu", dev["g"], dev["u"], dev["o"], n=64 * 1000 - 3)  # vec + scalar tail


def test_plan_replay_matches_direct(hip):
    s, d, e = _inputs(5)
    n_rot, inv_h = ops.rope_inv_freq(s.head_dim, None, s.theta)
    inv = DA.from_numpy(inv_h)

    def fresh():
        dev = {k: DA.from_numpy(v) for k, v in d.items()}
        dev["tab"] = DA.from_numpy(e["table"])
        dev["ids"] = DA.from_numpy(e["ids"])
        dev["emb"] = DA.empty((64, s.hidden))
        dev["h"] = DA.empty((64, s.hidden))
        dev["o"] = DA.from_numpy(np.zeros((64, 1000), np.float32))
        return dev

    direct = fresh()
    _record_or_run(s, direct, e, inv)
    planned = fresh()
    plan = Plan()
    with plan:
        _record_or_run(s, planned, e, inv)
    assert len(plan) == 5  # gather, norm, rope, act vec + act tail
    # nothing ran while recording
    assert bits_equal(planned["q"].numpy(), d["q"])
    assert not planned["o"].numpy().any()
    stream = Stream()
    starts, stops = [Event() for _ in range(5)], [Event() for _ in range(5)]
    plan.launch(stream, plan.event_arrays(starts, stops))
    stream.synchronize()
    for key in ("emb", "h", "q", "k", "o"):
        assert bits_equal(planned[key].numpy(), direct[key].numpy()), key
    assert all(a.elapsed_ms(b) > 0 for a, b in zip(starts, stops))
    # a second replay repeats the same kernels (rope is in place: rotates again)
    plan.launch(stream)
    _record_or_run(s, direct, e, inv)
    stream.synchronize()
    for key in ("emb", "h", "q", "k", "o"):
        assert bits_equal(planned[key].numpy(), direct[key].numpy()), key
    plan.destroy()
    stream.destroy()


def test_plan_refusal_is_reported_at_record_time(hip):
    plan = Plan()
    x = DA.empty((4, 8))
    with pytest.raises(Exception):
        with plan:
            ops.rmsnorm(x, None, x, 4, 16, 1e-6)   # buffer too small: host check
    assert len(plan) == 0
    plan.destroy()


def test_plan_keeps_its_workspace_after_a_larger_call(hip):
    """A plan that recorded a DeltaNet scan (129 tokens: the chunked form, with
    a workspace) holds that workspace; a later, larger scan outside the plan
    replaces the shared buffer, and replaying the plan still reproduces the
    direct call bit for bit (it writes its own, still-allocated buffer)."""
    rng = np.random.default_rng(17)
    T, n_k, n_v, d = 129, 2, 4, 128
    host = [rng.standard_normal(s).astype(np.float32) for s in
            ((T, n_k, d), (T, n_k, d), (T, n_v, d), (T, n_v), (T, n_v))]
    a_log = (-np.abs(rng.standard_normal(n_v)) * 0.5).astype(np.float32)
    dt_bias = rng.standard_normal(n_v).astype(np.float32)
    st0 = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
    dev = [DA.from_numpy(h) for h in host] + [DA.from_numpy(a_log), DA.from_numpy(dt_bias)]

    def scan(state, outs, plan=None):
        ops.ssm_scan(*dev, state, outs, T, n_k, n_v, d, d ** -0.5)

    want_state, want_out = DA.from_numpy(st0), DA.empty((T, n_v, d))
    scan(want_state, want_out)
    p_state, p_out = DA.from_numpy(st0), DA.empty((T, n_v, d))
    plan = Plan()
    with plan:
        scan(p_state, p_out)
    recorded = ops._ssm_ws.buf
    assert any(b is recorded for b in plan._held)
    # a larger scan outside the plan grows the shared workspace
    Tb = 700
    big = [DA.from_numpy(rng.standard_normal(s).astype(np.float32)) for s in
           ((Tb, n_k, d), (Tb, n_k, d), (Tb, n_v, d), (Tb, n_v), (Tb, n_v))]
    ops.ssm_scan(*big, dev[5], dev[6], DA.from_numpy(st0), DA.empty((Tb, n_v, d)), Tb, n_k,
                 n_v, d, d ** -0.5)
    assert ops._ssm_ws.buf is not recorded and recorded.nbytes > 0
    stream = Stream()
    plan.launch(stream)
    stream.synchronize()
    assert bits_equal(p_out.numpy(), want_out.numpy())
    assert bits_equal(p_state.numpy(), want_state.numpy())
    plan.destroy()
    stream.destroy()


def test_split_gemm_workspace_is_one_buffer_for_alternating_widths(hip):
    """A prefill layer alternates 4096- and 14336-column GEMMs: the split
    GEMM's workspace is allocated for the widest and then reused (no free and
    reallocate per switch); results are unchanged by the reuse."""
    rng = np.random.default_rng(23)
    n_tok, n_rows = 64, 32
    outs = {}
    for n_cols in (4096, 14336, 4096, 14336):
        w = W.make_table(W.Q4_K, n_rows * n_cols // 256, rng) if n_cols not in outs else \
            outs[n_cols][0]
        x = rng.standard_normal((n_tok, n_cols)).astype(np.float32) if n_cols not in outs \
            else outs[n_cols][1]
        y = DA.empty((n_tok, n_rows))
        ops.matvec(W.Q4_K, DA.from_numpy(w), DA.from_numpy(x), y, n_rows, n_cols, n_tok)
        if n_cols in outs:
            assert bits_equal(y.numpy(), outs[n_cols][2])
            assert ops._gemm_ws.buf is held
        else:
            outs[n_cols] = (w, x, y.numpy())
            held = ops._gemm_ws.buf
    assert held.nbytes >= _lib_ws(14336, n_tok)


def _lib_ws(n_cols, n_tok):
    from aero_amd import _lib
    return int(_lib.lib().aero_hip_matmul_workspace(W.Q4_K, n_cols, n_tok))


def test_host_pointer_abi_refuses_inside_a_plan(hip):
    """The reference-compatible host ABI runs and copies back at once; inside
    plan recording it refuses (status 0 and a reason) instead of recording a
    kernel over its staging arena and returning the input unmodified."""
    import ctypes
    from aero_amd import _lib

    L = _lib.lib()
    v = np.linspace(-3, 3, 64).astype(np.float32)
    before = v.copy()
    plan = Plan()
    with plan:
        ok = L.aero_tensor_silu(v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), v.size)
        msg = _lib.last_error()
    assert ok == 0 and "plan" in msg
    assert len(plan) == 0 and bits_equal(v, before)
    plan.destroy()
