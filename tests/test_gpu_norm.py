"""GPU parity: RMSNorm (plain, (1+w), weightless, L2) and the gated norm*silu
against the oracle (oracle/cpuref.c restating src/tensor.cpp:128-164 and
src/ssm.cpp:327-343), at the layer shapes and at edge shapes.

Tolerance: the reference's RTOL = 1e-5 relative to the reference's scale
(tests/test_transformer_native.py:34-37,52-61); the GPU differs from the
serial fp32 sum only in summation order.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, golden, rel_to_scale
from aero_amd import ops
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA

pytestmark = pytest.mark.gpu

NORM_SHAPES = ["qwen2_0p5b_decode", "llama3_8b_prefill", "gemma3_4b_prefill",
               "qwen3next_hybrid", "llama3_70b_decode64", "llama3_70b_prefill16k"]


def gpu_norm(x, w, eps, unit_offset=False, l2=False, in_place=False):
    cols = x.shape[-1]
    rows = x.size // cols
    dx = DA.from_numpy(x)
    dw = None if w is None else DA.from_numpy(w)
    dout = dx if in_place else DA.empty(x.shape)
    ops.rmsnorm(dx, dw, dout, rows, cols, eps, unit_offset=unit_offset, l2=l2)
    return dout.numpy()


@pytest.mark.parametrize("name", NORM_SHAPES)
def test_rmsnorm_layer_shapes(hip, oracle, name):
    s = W.SHAPES[name]
    d = W.rmsnorm_inputs(s)
    print(f"rmsnorm {name} {d['x'].shape} unit_offset={d['unit_offset']}", flush=True)
    got = gpu_norm(d["x"], d["w"], d["eps"], d["unit_offset"])
    want = oracle.rmsnorm_rows(d["x"], d["w"], d["eps"], d["unit_offset"])
    r = rel_to_scale(got, want)
    assert r <= RTOL, r
    # in place (out aliases x) gives the same bits
    assert bits_equal(gpu_norm(d["x"], d["w"], d["eps"], d["unit_offset"], in_place=True), got)


def test_rmsnorm_weightless_is_ones_bitwise(hip, oracle):
    rng = np.random.default_rng(1)
    for cols in (16, 64, 896, 4096, 5000, 6):
        x = rng.standard_normal((5, cols)).astype(np.float32)
        a = gpu_norm(x, None, 1e-6)
        b = gpu_norm(x, np.ones(cols, np.float32), 1e-6)
        assert bits_equal(a, b), cols  # tests/test_transformer_cpp.cpp:289-294
        assert rel_to_scale(a, oracle.rmsnorm_rows(x, None, 1e-6)) <= RTOL


def test_unit_offset_is_composition_bitwise(hip):
    """(1+w) is rms_norm(x, np.float32(1) + w): bit-identical to passing 1+w."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 2560)).astype(np.float32)
    w = (rng.standard_normal(2560) * 0.1).astype(np.float32)
    assert bits_equal(gpu_norm(x, w, 1e-6, unit_offset=True),
                      gpu_norm(x, np.float32(1) + w, 1e-6))


def test_l2norm(hip, oracle):
    rng = np.random.default_rng(3)
    for rows, cols in ((6, 16), (4, 128), (3, 4096), (2, 33)):
        x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
        w = (rng.standard_normal(cols) + 2).astype(np.float32)
        assert rel_to_scale(gpu_norm(x, w, 1e-6, l2=True), oracle.l2norm_rows(x, w, 1e-6)) <= RTOL
        assert rel_to_scale(gpu_norm(x, None, 1e-6, l2=True),
                            oracle.l2norm_rows(x, None, 1e-6)) <= RTOL
    # the eps floor bites below ||x|| = eps (tests/test_tensor_native.py:154-181)
    tiny = np.full((1, 64), 1e-9, np.float32)
    got = gpu_norm(tiny, None, 1e-6, l2=True)
    assert abs(np.linalg.norm(got.astype(np.float64)) - 8e-9 / 1e-6) / (8e-9 / 1e-6) < 1e-3


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 3), (2, 7), (5, 17), (4, 100), (2, 4097),
                                       (1, 40000), (33, 64), (300, 12), (1, 131072)])
def test_rmsnorm_edge_shapes(hip, oracle, rows, cols):
    rng = np.random.default_rng(rows * 100003 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    assert rel_to_scale(gpu_norm(x, w, 1e-6), oracle.rmsnorm_rows(x, w, 1e-6)) <= RTOL


def test_rmsnorm_unaligned_pointer(hip, oracle):
    """A 4-byte offset view takes the scalar kernel with the same arithmetic."""
    rng = np.random.default_rng(5)
    rows, cols = 6, 256
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    buf = DA.empty(rows * cols + 4)
    xv = buf.view((rows, cols), offset_bytes=4)
    xv.copy_from(x)
    out = DA.empty((rows, cols))
    ops.rmsnorm(xv, DA.from_numpy(w), out, rows, cols, 1e-6)
    assert rel_to_scale(out.numpy(), oracle.rmsnorm_rows(x, w, 1e-6)) <= RTOL


def test_rmsnorm_zero_rows(hip):
    x = DA.empty((0, 64))
    ops.rmsnorm(x, None, x, 0, 64, 1e-6)


def test_rmsnorm_ones_in_weight_out(hip):
    """tests/test_tensor.cpp:98-104: ones in -> weight out."""
    w = np.linspace(0.5, 2.0, 64, dtype=np.float32)
    got = gpu_norm(np.ones((3, 64), np.float32), w, 1e-6)
    assert np.allclose(got, w[None, :], rtol=1e-5, atol=0)


def test_rmsnorm_golden(hip):
    g = golden("ref_vectors.npz")
    assert rel_to_scale(gpu_norm(g["norm_x"], g["norm_w"], 1e-6), g["rms_out"]) <= RTOL
    assert rel_to_scale(gpu_norm(g["norm_x"], None, 1e-6), g["rms_out_noweight"]) <= RTOL
    assert rel_to_scale(gpu_norm(g["norm_x"], g["norm_w"], 1e-6, l2=True), g["l2_out"]) <= RTOL
    assert rel_to_scale(gpu_norm(g["rms4096_x"], g["rms4096_w"], 1e-5), g["rms4096_out"]) <= RTOL


# ------------------------------------------------------------ gated norm
def gpu_gated(x, z, w, eps, group=None):
    inner = x.shape[-1]
    rows = x.size // inner
    out = DA.empty(x.shape)
    ops.gated_rmsnorm_silu(DA.from_numpy(x), DA.from_numpy(z), DA.from_numpy(w), out, rows,
                           inner, eps, group=group)
    return out.numpy()


@pytest.mark.parametrize("group", [None, 128])
def test_gated_norm_qwen3next(hip, oracle, group):
    s = W.SHAPES["qwen3next_hybrid"]
    d = W.gated_inputs(s)
    print(f"gated norm {d['x'].shape} group={group}", flush=True)
    got = gpu_gated(d["x"], d["z"], d["w"], d["eps"], group)
    want = oracle.gated_rmsnorm_silu(d["x"], d["z"], d["w"], d["eps"], group)
    assert rel_to_scale(got, want) <= RTOL


@pytest.mark.parametrize("rows,inner,d,group", [(3, 12, 4, 12), (2, 12, 4, 6), (5, 48, 16, 16),
                                                 (2, 30, 6, 30), (4, 4096, 128, 4096),
                                                 (1, 256, 128, 64)])
def test_gated_norm_edge(hip, oracle, rows, inner, d, group):
    rng = np.random.default_rng(inner + rows)
    x = rng.standard_normal((rows, inner)).astype(np.float32)
    z = rng.standard_normal((rows, inner)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    got = gpu_gated(x, z, w, 1e-6, group)
    assert rel_to_scale(got, oracle.gated_rmsnorm_silu(x, z, w, 1e-6, group)) <= RTOL


def test_gated_norm_invariant_unit_rms(hip):
    """w = 1 and z -> +inf (silu(z) = z): out/z has unit RMS over each group."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    z = np.full_like(x, 60.0)
    w = np.ones(128, np.float32)
    got = gpu_gated(x, z, w, 1e-6)
    r = (got.astype(np.float64) / 60.0)
    rms = np.sqrt((r * r).mean(axis=1))
    assert np.allclose(rms, 1.0, atol=1e-5)
