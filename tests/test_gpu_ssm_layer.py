"""GPU parity: the device-resident gated-DeltaNet layer (aero_amd.ssm_layer,
aero_ssm_forward_q of src/ssm.cpp:262-352) against the oracle's composition
of the same layer (oracle.cpuref.ssm_forward, itself checked against the
compiled reference in test_oracle.py).

Calls run in sequence on one SsmStep, carrying the recurrent state and the
conv history: a prompt (the chunked scan from 128 tokens), then decode calls.
Every call's output and the state after it: <= 1e-5 of scale (the GPU sums
its dots in another order, and the chunked scan re-associates the delta rule).
"""
import numpy as np
import pytest

from conftest import RTOL, rel_to_scale
from aero_amd import ssm_layer as S
from aero_amd import workloads as W
from aero_amd.device import Plan, Stream

pytestmark = pytest.mark.gpu


def run_chain(oracle, cfg, seed, calls, fusions=None):
    wts = S.SsmWeights(cfg, seed=seed)
    step = S.SsmStep(cfg, wts, max_tokens=max(calls), fusions=fusions)
    h = wts.host
    case = dict(dts=list(cfg.wtypes), weights=[h[n] for n in S.PROJ], a_log=h["a_log"],
                dt_bias=h["dt_bias"], conv1d=h["conv1d"], norm=h["norm"], n_k=cfg.n_k,
                d=cfg.head_dim, inner=cfg.inner, eps=cfg.eps, norm_eps=cfg.norm_eps)
    K = cfg.conv_kernel
    tail, tl = np.zeros((K - 1, cfg.qkv), np.float32), 0
    st = np.zeros((cfg.n_v, cfg.head_dim, cfg.head_dim), np.float32)
    rng = np.random.default_rng(seed + 1)
    for i, T in enumerate(calls):
        x = rng.standard_normal((T, cfg.hidden)).astype(np.float32)
        print(f"  call {i}: {T} tokens", flush=True)
        step.x.view((T, cfg.hidden)).copy_from(x)
        step.forward(T)
        want, tail, tl, st = oracle.ssm_forward(x, tail=tail, tail_len=tl, state=st, **case)
        got = step.out.view((T, cfg.hidden)).numpy()
        e_out, e_st = rel_to_scale(got, want), rel_to_scale(step.state.numpy(), st)
        print(f"    out {e_out:.2e} state {e_st:.2e}", flush=True)
        assert e_out <= RTOL and e_st <= RTOL, (i, T, e_out, e_st)
        assert step.tail_len == tl


@pytest.mark.parametrize("name,cfg,calls", [
    # Qwen3-Next's heads (16 key, 32 value, d 128) at a narrower hidden size
    ("qwen3next_heads_q4k", S.SsmConfig(512, 16, 32, 128, 4, (W.Q4_K,) * 5), (200, 1, 1, 3)),
    # mixed types: Q4_K projections with Q8_0 gate inputs (two launches for x)
    ("mixed_q4k_q8_0", S.SsmConfig(1024, 4, 8, 128, 4, (W.Q4_K, W.Q4_K, W.Q8_0, W.Q8_0, W.Q4_K)),
     (130, 2, 1)),
    ("d64_q8_0", S.SsmConfig(256, 2, 4, 64, 4, (W.Q8_0,) * 5), (1, 140, 1, 17)),
    ("d256_q6k", S.SsmConfig(256, 1, 2, 256, 4, (W.Q6_K, W.Q6_K, W.Q8_0, W.Q8_0, W.Q6_K)),
     (129, 1)),
    ("kernel3_short", S.SsmConfig(256, 2, 2, 128, 3, (W.Q8_0,) * 5), (1, 1, 5, 40)),
])
def test_ssm_layer_vs_oracle(hip, oracle, name, cfg, calls):
    print(f"ssm layer {name}", flush=True)
    run_chain(oracle, cfg, 5 + len(name), calls)


def test_ssm_layer_decode_conv_unfolded(hip, oracle):
    """The same chain with the conv as its own launch at one token."""
    cfg = S.SsmConfig(512, 4, 8, 128, 4, (W.Q4_K,) * 5)
    run_chain(oracle, cfg, 17, (1, 1, 40, 1, 1), fusions={"conv_gemm": False})


def test_ssm_layer_plan_replay(hip, oracle):
    """The decode call recorded once as a plan and replayed three times, each
    replay a new token against the state the previous one left; every replay
    equals the oracle's chain."""
    cfg = S.SsmConfig(512, 4, 8, 128, 4, (W.Q4_K,) * 5)
    wts = S.SsmWeights(cfg, seed=3)
    step = S.SsmStep(cfg, wts, max_tokens=64)
    h = wts.host
    case = dict(dts=list(cfg.wtypes), weights=[h[n] for n in S.PROJ], a_log=h["a_log"],
                dt_bias=h["dt_bias"], conv1d=h["conv1d"], norm=h["norm"], n_k=cfg.n_k,
                d=cfg.head_dim, inner=cfg.inner, eps=cfg.eps, norm_eps=cfg.norm_eps)
    rng = np.random.default_rng(9)
    tail, tl = np.zeros((3, cfg.qkv), np.float32), 0
    st = np.zeros((cfg.n_v, cfg.head_dim, cfg.head_dim), np.float32)
    x = rng.standard_normal((40, cfg.hidden)).astype(np.float32)
    step.x.view((40, cfg.hidden)).copy_from(x)
    step.forward(40)       # a prompt: the history is kernel - 1 rows from here on
    _, tail, tl, st = oracle.ssm_forward(x, tail=tail, tail_len=tl, state=st, **case)
    stream = Stream()
    plan = Plan()
    with plan:
        step.forward(1, stream=stream)
    for i in range(3):
        x = rng.standard_normal((1, cfg.hidden)).astype(np.float32)
        step.x.view((1, cfg.hidden)).copy_from(x)
        plan.launch(stream)
        stream.synchronize()
        want, tail, tl, st = oracle.ssm_forward(x, tail=tail, tail_len=tl, state=st, **case)
        e = rel_to_scale(step.out.view((1, cfg.hidden)).numpy(), want)
        print(f"  replay {i}: out {e:.2e}", flush=True)
        assert e <= RTOL
        assert rel_to_scale(step.state.numpy(), st) <= RTOL
    plan.destroy()
    stream.destroy()


def test_ssm_layer_decode_launches(hip):
    """Decode is three launches (projections of x with the conv and silu on
    the qkv rows in their epilogue, scan, gated norm in the output
    projection's GEMV); four with the conv_gemm fusion off (the conv writing
    its own history) or with norm_gemm off (the gated norm its own launch)."""
    cfg = S.SsmConfig(512, 4, 8, 128, 4, (W.Q4_K,) * 5)
    wts = S.SsmWeights(cfg, seed=1)
    for fus, want in (({}, 3), ({"conv_gemm": False}, 4), ({"norm_gemm": False}, 4),
                      ({"conv_gemm": False, "norm_gemm": False}, 5)):
        step = S.SsmStep(cfg, wts, max_tokens=8, fusions=fus)
        step.forward(4)
        plan = Plan()
        with plan:
            step.forward(1)
        assert len(plan) == want, (fus, len(plan))
        plan.destroy()


def test_ssm_layer_refusals(hip):
    with pytest.raises(ValueError, match="head dim"):
        S.SsmStep(S.SsmConfig(256, 1, 1, 32, 4, (W.Q8_0,) * 5),
                  S.SsmWeights(S.SsmConfig(256, 1, 1, 32, 4, (W.Q8_0,) * 5)), 8)
    cfg = S.SsmConfig(256, 2, 2, 64, 4, (W.Q8_0,) * 5)
    step = S.SsmStep(cfg, S.SsmWeights(cfg), max_tokens=8)
    with pytest.raises(ValueError, match="tokens"):
        step.forward(9)


def _conv_fold_admits(t, hidden):
    bv, bb = W.BLOCK[t]
    return hidden % bv == 0 and (hidden // bv * bb) % 16 == 0


PROJ_CONV_CASES = [(W.Q4_K, h, tl) for h in (1024, 2048) for tl in (0, 1, 2, 3)] + [
    (t, h, tl) for t in (W.Q4_K, W.Q8_0, W.Q5_K, W.Q6_K, W.IQ4_XS)
    for h in (1024, 2048, 4096, 5120) for tl in (0, 3)
    if _conv_fold_admits(t, h) and not (t == W.Q4_K and h <= 2048)]


@pytest.mark.parametrize("t,hidden,tail_len", PROJ_CONV_CASES)
def test_ssm_proj_conv_equals_separate_launches(hip, t, hidden, tail_len):
    """aero_hip_ssm_proj_conv against the same projections (norm_matmul with
    no norm) followed by the conv with silu, at every history length, for
    every type the layer's conv fold admits and for rows that take each
    GEMV form (quarter and half wave up to 2048 columns, a whole wave up to
    4096, the pipelined form beyond): the conv output and the moved history
    bit for bit (the same arithmetic in the same order), the other
    projections likewise."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray as DA
    print(f"proj_conv type={t} hidden={hidden} tail_len={tail_len}", flush=True)
    cfg = S.SsmConfig(hidden, 2, 4, 64, 4, (t,) * 5)
    wts = S.SsmWeights(cfg, seed=tail_len)
    h, d = wts.host, wts.dev
    rng = np.random.default_rng(71 + tail_len)
    x = DA.from_numpy(rng.standard_normal((1, hidden)).astype(np.float32))
    tail0 = rng.standard_normal((3, cfg.qkv)).astype(np.float32)
    names = S.PROJ[:4]
    rows = [cfg.shapes()[n][0] for n in names]
    ws = [d[n] for n in names]
    # separate launches
    ys_a = [DA.empty((1, r)) for r in rows]
    ops.norm_matmul(t, ws, x, ys_a, rows, hidden, 1, norm=False)
    tail_a, conv_a = DA.from_numpy(tail0), DA.empty((1, cfg.qkv))
    tl_a = ops.ssm_conv(ys_a[0], d["conv1d"], tail_a, tail_len, tail_a, conv_a, 1, cfg.qkv, 4,
                        silu=True)
    # one launch
    ys_b = [DA.empty((1, r)) for r in rows]
    tail_b, conv_b = DA.from_numpy(tail0), DA.empty((1, cfg.qkv))
    tl_b = ops.ssm_proj_conv(t, ws, x, ys_b, rows, hidden, d["conv1d"], tail_b, tail_len,
                             conv_b)
    assert tl_a == tl_b == min(3, tail_len + 1)
    assert np.array_equal(conv_a.numpy(), conv_b.numpy())
    assert np.array_equal(tail_a.numpy()[:tl_a], tail_b.numpy()[:tl_b])
    for ya, yb in zip(ys_a[1:], ys_b[1:]):
        assert np.array_equal(ya.numpy(), yb.numpy())
    with pytest.raises(Exception, match="history"):
        ops.ssm_proj_conv(t, ws, x, ys_b, rows, hidden, d["conv1d"], tail_b, 4, conv_b)


def test_ssm_proj_conv_refuses_overlaps(hip):
    """conv_out and the history tail are written by single lanes while every
    workgroup reads x: overlapping x, each other or another output is
    refused on the host, before any launch."""
    from aero_amd import _lib, ops
    from aero_amd.device import DeviceArray as DA
    cfg = S.SsmConfig(1024, 2, 4, 64, 4, (W.Q4_K,) * 5)
    wts = S.SsmWeights(cfg, seed=5)
    d = wts.dev
    names = S.PROJ[:4]
    rows = [cfg.shapes()[n][0] for n in names]
    C = rows[0]
    ws = [d[n] for n in names]
    x = DA.from_numpy(np.ones((1, 1024), np.float32))
    tail, conv = DA.empty((3, C)), DA.empty((1, C))
    big = DA.empty((4 * C,))
    shared = DA.empty((max(C, rows[1]),))
    ys = [DA.empty((1, r)) for r in rows]
    ys_shared = [ys[0], shared.view((1, rows[1]))] + ys[2:]
    cases = {
        "conv_out inside the tail": (ys, tail, tail.view((1, C), offset_bytes=8)),
        "tail over conv_out": (ys, big, big.view((1, C), offset_bytes=4 * C)),
        "conv_out over x": (ys, tail, x.view((1, C))),
        "conv_out over y[1]": (ys_shared, tail, shared.view((1, C))),
    }
    for what, (yy, tl, cv) in cases.items():
        print(f"proj_conv overlap refusal: {what}", flush=True)
        with pytest.raises(_lib.AeroHipError, match="overlap"):
            ops.ssm_proj_conv(W.Q4_K, ws, x, yy, rows, 1024, d["conv1d"], tl, 0, cv)
    # apart: accepted (returns the history's new length)
    assert ops.ssm_proj_conv(W.Q4_K, ws, x, ys, rows, 1024, d["conv1d"], tail, 0, conv) == 1


def test_ssm_layer_plan_refuses_short_history(hip):
    """A plan recorded before the conv history is full would replay the short
    history length forever: forward refuses to record then."""
    cfg = S.SsmConfig(512, 4, 8, 128, 4, (W.Q4_K,) * 5)
    step = S.SsmStep(cfg, S.SsmWeights(cfg, seed=2), max_tokens=8)
    plan = Plan()
    with pytest.raises(ValueError, match="history"):
        with plan:
            step.forward(1)
    plan.destroy()
    step.forward(3)          # three rows of history now
    plan = Plan()
    with plan:
        step.forward(1)
    assert len(plan) > 0
    plan.destroy()
