"""GPU parity: act*mul (SwiGLU, GeGLU erf / tanh), unary silu / gelu and the
plain product against the oracle (oracle/cpuref.c restating src/tensor.cpp:
47-59,104-125) and against float64 closed forms.
"""
import math

import numpy as np
import pytest

from conftest import RTOL, bits_equal, golden, rel_to_scale
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

KIND = {"silu": 0, "gelu": 1, "gelu_tanh": 2, "identity": 3}


def gpu_act(kind, g, u=None, alias=None):
    dg = DA.from_numpy(g)
    du = None if u is None else DA.from_numpy(u)
    out = dg if alias == "gate" else (du if alias == "up" else DA.empty(g.shape))
    ops.act_mul(KIND[kind], dg, du, out, g.size)
    return out.numpy()


@pytest.mark.parametrize("name", ["qwen2_0p5b_decode", "llama3_8b_prefill", "gemma3_4b_prefill",
                                  "qwen3next_hybrid", "llama3_70b_decode64"])
def test_act_mul_layer_shapes(hip, oracle, name):
    s = W.SHAPES[name]
    d = W.act_inputs(s)
    kinds = [d["act"]] + (["gelu"] if d["act"] == "gelu_tanh" else [])
    for kind in kinds:
        print(f"act_mul {name} {kind} {d['gate'].shape}", flush=True)
        got = gpu_act(kind, d["gate"], d["up"])
        want = oracle.act_mul(KIND[kind], d["gate"], d["up"])
        assert rel_to_scale(got, want) <= RTOL


def test_act_mul_70b_prefill_full_size(hip, oracle):
    """16384 x 28672 (1.9 GB per tensor, byte offsets past 2^31): inputs are 61
    random rows repeated, so every output row is checked against the oracle's
    row for it."""
    s = W.SHAPES["llama3_70b_prefill16k"]
    base = W.act_inputs(s, rows=61)
    R, F = s.n_tok, s.ffn
    g = np.resize(base["gate"], (R, F))
    u = np.resize(base["up"], (R, F))
    want = oracle.act_mul(0, base["gate"], base["up"])
    got = gpu_act("silu", g, u)
    del g, u
    idx = np.arange(R) % 61
    worst = 0.0
    for r0 in range(0, R, 2048):
        blk = got[r0:r0 + 2048]
        ref = want[idx[r0:r0 + 2048]]
        worst = max(worst, float(np.abs(blk.astype(np.float64) - ref).max()))
    assert worst / float(np.abs(want).max()) <= RTOL


@pytest.mark.parametrize("kind", ["silu", "gelu", "gelu_tanh"])
def test_unary(hip, oracle, kind):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(100003) * 4).astype(np.float32)
    assert rel_to_scale(gpu_act(kind, x), oracle.act(KIND[kind], x)) <= RTOL


def test_mul(hip, oracle):
    rng = np.random.default_rng(12)
    a = rng.standard_normal(77777).astype(np.float32)
    b = rng.standard_normal(77777).astype(np.float32)
    assert bits_equal(gpu_act("identity", a, b), a * b)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 1023, 1024, 1025, 4099, 262147])
def test_odd_lengths(hip, oracle, n):
    rng = np.random.default_rng(n)
    g = rng.standard_normal(n).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    for kind in ("silu", "gelu", "gelu_tanh"):
        assert rel_to_scale(gpu_act(kind, g, u), oracle.act_mul(KIND[kind], g, u)) <= RTOL


def test_aliasing_and_unaligned(hip, oracle):
    rng = np.random.default_rng(13)
    g = rng.standard_normal(5000).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    want = oracle.act_mul(0, g, u)
    assert rel_to_scale(gpu_act("silu", g, u, alias="gate"), want) <= RTOL
    assert rel_to_scale(gpu_act("silu", g, u, alias="up"), want) <= RTOL
    # misaligned views (offset 4 bytes) take the scalar kernel
    bg, bu, bo = DA.empty(5001), DA.empty(5001), DA.empty(5001)
    vg, vu, vo = (b.view((5000,), offset_bytes=4) for b in (bg, bu, bo))
    vg.copy_from(g)
    vu.copy_from(u)
    ops.act_mul(0, vg, vu, vo, 5000)
    assert rel_to_scale(vo.numpy(), want) <= RTOL


def test_closed_forms(hip):
    """erf GELU against math.erf, tanh GELU and silu against float64 closed forms."""
    z = np.linspace(-8, 8, 4001, dtype=np.float32)
    z64 = z.astype(np.float64)
    gelu_exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in z64])
    tanh_exact = 0.5 * z64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (z64 + 0.044715 * z64 ** 3)))
    silu_exact = z64 / (1 + np.exp(-z64))
    # A&S 7.1.26 error < 1.5e-7 times |z|/2 plus fp32 rounding
    assert np.abs(gpu_act("gelu", z) - gelu_exact).max() < 2e-6
    assert rel_to_scale(gpu_act("gelu_tanh", z), tanh_exact) < 1e-6
    assert rel_to_scale(gpu_act("silu", z), silu_exact) < 1e-6
    # gelu is the erf form, not tanh (tests/test_tensor_native.py:118-126)
    for xv in (1.0, 3.0, -2.5):
        got = float(gpu_act("gelu", np.array([xv], np.float32))[0])
        want = 0.5 * xv * (1.0 + math.erf(xv / math.sqrt(2.0)))
        tanh = 0.5 * xv * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (xv + 0.044715 * xv ** 3)))
        assert abs(got - want) < 1e-6 and abs(got - tanh) > 1e-7


def test_act_golden(hip):
    g = golden("ref_vectors.npz")
    z, up = g["act_z"], g["act_up"]
    assert rel_to_scale(gpu_act("silu", z), g["silu_out"]) <= RTOL
    assert rel_to_scale(gpu_act("gelu", z), g["gelu_out"]) <= RTOL
    assert rel_to_scale(gpu_act("silu", z, up), g["swiglu_out"]) <= RTOL
    assert bits_equal(gpu_act("identity", z, up), g["mul_out"])
