"""GPU: the alternative launch shapes the AERO_HIP_TUNE knobs select compute
what the default shapes compute.

- `norm_loop` (a persistent grid of a few workgroups per CU, weights held in
  registers, the next row's loads issued before this row's stores) keeps the
  per-row kernel's lanes-per-row split and summation order: bit-identical.
- `act_grid` (a persistent act·mul grid): bit-identical.
- `norm_vmax` 16 / 32 (one or two waves a row, 16 or 32 float4 a lane)
  changes the summation order: within the reference's RTOL of the oracle,
  and x + d of the residual form bit-exact.
- the store-only fill writes exactly its value.
Knobs are dropped again after every case, so later tests see the defaults.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA, tune_set

pytestmark = pytest.mark.gpu


class knobs:
    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        for k, v in self.kv.items():
            tune_set(k, v)

    def __exit__(self, *exc):
        for k in self.kv:
            tune_set(k, None)


def run_norm(mode, x, z, w, eps, unit=False, group=None):
    rows, cols = x.shape
    dx, dz = DA.from_numpy(x), DA.from_numpy(z)
    if mode == "gated":
        out = DA.empty(x.shape)
        ops.gated_rmsnorm_silu(dx, dz, DA.from_numpy(w), out, rows, cols, eps, group=group)
        return out.numpy(), None
    dw = None if w is None else DA.from_numpy(w)
    h = DA.empty(x.shape)
    if mode == "plain":
        ops.rmsnorm(dx, dw, h, rows, cols, eps, unit_offset=unit)
        return h.numpy(), None
    ops.add_rmsnorm(dx, dz, dw, h, rows, cols, eps, unit_offset=unit)
    return h.numpy(), dx.numpy()


CASES = [("plain", 3000, 4096, {}), ("plain", 2049, 8192, {}),
         ("plain", 5000, 2560, {"unit": True}), ("plain", 4000, 2048, {"weight": False}),
         ("plain", 1500, 896, {}), ("resid", 3000, 4096, {}),
         ("resid", 2500, 2560, {"unit": True}), ("resid", 2049, 8192, {}),
         ("gated", 3000, 4096, {}), ("gated", 1000, 4096, {"group": 128}),
         ("gated", 2000, 2048, {})]


def inputs(mode, rows, cols, weight=True, seed=0):
    rng = np.random.default_rng(seed + rows + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    z = rng.standard_normal((rows, cols), dtype=np.float32)
    if mode == "gated":
        w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    else:
        w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32) if weight else None
    return x, z, w


@pytest.mark.parametrize("mode,rows,cols,kw", CASES)
@pytest.mark.parametrize("per_cu", [1, 2])
def test_persistent_norm_is_bitwise(hip, mode, rows, cols, kw, per_cu):
    x, z, w = inputs(mode, rows, cols, kw.get("weight", True))
    eps = 1e-6 if mode == "gated" else 1e-5
    args = dict(unit=kw.get("unit", False)) if mode != "gated" else dict(group=kw.get("group"))
    print(f"norm_loop={per_cu} {mode} {rows}x{cols} {kw}", flush=True)
    a, ax = run_norm(mode, x, z, w, eps, **args)
    with knobs(norm_loop=per_cu):
        b, bx = run_norm(mode, x, z, w, eps, **args)
    assert bits_equal(a, b)
    if ax is not None:
        assert bits_equal(ax, bx)


@pytest.mark.parametrize("mode,rows,cols,kw", CASES[:2] + CASES[5:6] + CASES[7:9])
@pytest.mark.parametrize("vmax", [16, 32])
def test_wide_rows_vs_oracle(hip, oracle, mode, rows, cols, kw, vmax):
    x, z, w = inputs(mode, rows, cols, kw.get("weight", True), seed=1)
    rows = min(rows, 300)
    x, z = x[:rows], z[:rows]
    print(f"norm_vmax={vmax} {mode} {rows}x{cols}", flush=True)
    with knobs(norm_vmax=vmax):
        got, gx = run_norm(mode, x, z, w, 1e-6 if mode == "gated" else 1e-5,
                           **({"group": None} if mode == "gated" else {}))
    if mode == "gated":
        want = oracle.gated_rmsnorm_silu(x, z, w, 1e-6)
    elif mode == "plain":
        want = oracle.rmsnorm_rows(x, w, 1e-5)
    else:
        s = (x + z).astype(np.float32)
        assert bits_equal(gx, s)
        want = oracle.rmsnorm_rows(s, w, 1e-5)
    assert rel_to_scale(got, want) <= RTOL


@pytest.mark.parametrize("n", [4 * 1000003, 512 * 14336, 4 * 64 * 512 * 3 + 8])
@pytest.mark.parametrize("bs", [64, 256])
def test_persistent_act_is_bitwise(hip, n, bs):
    rng = np.random.default_rng(n)
    g = rng.standard_normal(n, dtype=np.float32)
    u = rng.standard_normal(n, dtype=np.float32)

    def run():
        o = DA.empty(n)
        ops.act_mul("silu", DA.from_numpy(g), DA.from_numpy(u), o)
        return o.numpy()

    print(f"act_grid n={n} bs={bs}", flush=True)
    with knobs(act_bs=bs):
        a = run()
    with knobs(act_grid=2, act_bs=bs):
        b = run()
    assert bits_equal(a, b)


def test_fill_writes_its_value(hip):
    for n in (4, 1024, 4 * 70001):
        d = DA.from_numpy(np.zeros(n + 4, np.float32))
        ops.fill_f32(d, 2.5, n)
        out = d.numpy()
        assert (out[:n] == np.float32(2.5)).all() and (out[n:] == 0).all(), n


def test_tune_set_refuses_empty_key(hip):
    assert hip.aero_hip_tune_set(b"", 1, 0) == 0


def test_gated_fast_form_within_tolerance_at_extremes(hip, oracle):
    """The gated norm multiplies by 1/denom and takes silu from the hardware
    exp and reciprocal: within RTOL of the reference's division form at large
    |z| (exp over- and underflow) and tiny rows."""
    rng = np.random.default_rng(9)
    for rows, inner in ((16, 4096), (3, 128), (64, 2048)):
        x = rng.standard_normal((rows, inner), dtype=np.float32) * 5
        z = (rng.standard_normal((rows, inner), dtype=np.float32) * 40).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        got, _ = run_norm("gated", x, z, w, 1e-6)
        assert rel_to_scale(got, oracle.gated_rmsnorm_silu(x, z, w, 1e-6)) <= RTOL
    assert W.SHAPES["qwen3next_hybrid"].gated
