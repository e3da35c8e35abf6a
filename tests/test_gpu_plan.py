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
