"""CPU: the C-ABI library loads and exports exactly what include/aero_hip.h
declares; the host-side logic (argument checks, refusals, host-only
arithmetic, the reference-shaped Python surface) behaves without a GPU.
Nothing here launches a kernel."""
import inspect
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, bits_equal
from aero_amd import _lib

HEADER = os.path.join(ROOT, "include", "aero_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aero_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.load()
    assert L is not None, _lib.unavailable_reason()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (aero_[a-z0-9_]+)$", out, flags=re.M))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing


def test_python_prototypes_match_header():
    assert sorted(_lib.PROTOTYPES) == declared_symbols()


def test_library_is_gfx950():
    """The device code bundled into our own build targets gfx950 only."""
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert b"amdgcn-amd-amdhsa--" + other not in blob


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "aero_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), f
                assert "cpuref" not in text, f


def test_host_only_entry_points_match_oracle():
    """aero_hip_rope_inv_freq is host arithmetic: bit-identical to the oracle's
    restatement of src/transformer.cpp:34-47."""
    from aero_amd import ops
    from oracle import cpuref as O
    for hd, nd, base, ff in ((128, None, 5e5, None), (256, 64, 1e7, None), (64, None, 1e6, None),
                             (64, 48, 1e4, None), (63, None, 1e4, None),
                             (64, None, 1e4, np.concatenate([np.ones(16, np.float32),
                                                             np.full(16, 1e30, np.float32)]))):
        n1, a = ops.rope_inv_freq(hd, nd, base, ff)
        n2, b = O.rope_inv_freq(hd, nd, base, ff)
        assert n1 == n2 and bits_equal(a, b)
    with pytest.raises(ValueError):
        ops.rope_inv_freq(64, None, 1e4, np.ones(3, np.float32))
    L = _lib.load()
    for t, bb, bv in ((8, 34, 32), (12, 144, 256), (14, 210, 256), (13, 176, 256), (0, 4, 1),
                      (1, 2, 1), (30, 2, 1), (99, 0, 0)):
        assert L.aero_dtype_block_bytes(t) == bb and L.aero_dtype_block_values(t) == bv
    assert 1 <= L.aero_hardware_threads() <= 8


def test_refusals_happen_before_device_work():
    """Bad arguments are refused (0 / -1) with a reason, with no GPU touched."""
    L = _lib.load()
    assert L.aero_hip_rmsnorm(None, None, None, 1, 4, 1e-6, 0, None) == 0
    assert "rmsnorm" in _lib.last_error()
    assert L.aero_hip_gated_rmsnorm_silu(1, 1, 1, 4, 1, 2, 12, 5, 1e-6, None) == 0  # 12 % 5
    assert L.aero_hip_act_mul(7, 1, 1, 1, 4, None) == 0
    assert "kind" in _lib.last_error()
    assert L.aero_hip_qk_norm_rope(1, None, 1, None, None, 0, None, None, 1e-6, 0, 1, 64, 128, 0,
                                   None, 1, None, None, 0, None) == 0          # n_rot > D
    assert L.aero_hip_qk_norm_rope(1, None, 1, None, None, 0, None, None, 1e-6, 0, 1, 64, 64, 0,
                                   None, 1, 1, 1, 4, None) == 0                # inv and table
    assert L.aero_hip_embed_gather(13, 1, 1 << 20, 10, 256, 1, 1, 0.0, 16, None, None) == 0
    assert L.aero_hip_embed_gather(12, 4, 100, 10, 256, 1, 1, 0.0, 16, None, None) == 0
    assert "table_bytes" in _lib.last_error()
    assert L.aero_hip_embed_gather(12, 4, 10 * 144, 10, 250, 1, 1, 0.0, 16, None, None) == 0
    assert L.aero_hip_dequant(23, 1, 1000, 16, 256, None) == 0
    assert L.aero_hip_dequant(12, 4, 100, 16, 256, None) == 0          # raw too short
    assert L.aero_tensor_silu(None, 4) == 0
    assert L.aero_tensor_rmsnorm(None, None, None, 0, 1e-6) == 0
    assert L.aero_tensor_l2norm(None, None, None, 4, 1e-6, 1) == 0
    assert L.aero_rope_tables(0, None, 0, 1e4, -1, None, 0, None, None) == -1
    assert L.aero_dequant_ref(23, None, 0, None, 256) == 0
    assert L.aero_hip_matvec(0, 4, 1 << 20, 16, 16, 4, 256, 1, None) == 0          # F32
    assert L.aero_hip_matvec(12, 4, 1 << 20, 16, 16, 4, 255, 1, None) == 0         # 255 % 256
    assert L.aero_hip_matvec(12, 4, 100, 16, 16, 4, 256, 1, None) == 0             # short W
    assert "w_bytes" in _lib.last_error()
    assert L.aero_matvec(0, None, None, None, 4, 16, 1) == 0
    assert L.aero_matmul(14, None, None, None, 2, 4, 255, 1) == 0
    assert L.aero_hip_plan_begin(None) == 0
    assert L.aero_hip_time_next_kernel(1, None) == 0


no_gpu = pytest.mark.skipif(_lib.available(), reason="a GPU is visible")


@no_gpu
def test_no_gpu_means_loud_unavailability():
    from aero_amd import native, ops, tensor_native, transformer_native
    from aero_amd.device import DeviceArray
    assert "device" in _lib.unavailable_reason()
    with pytest.raises(tensor_native.TensorLibUnavailable):
        tensor_native.silu(np.ones(4, np.float32))
    with pytest.raises(transformer_native.TransformerUnavailable):
        transformer_native.rmsnorm_rows(np.ones((2, 4), np.float32))
    with pytest.raises(native.KernelsUnavailable):
        native.dequant(8, bytes(34), (32,))
    with pytest.raises(_lib.AeroHipUnavailable):
        DeviceArray.empty(16)
    assert not tensor_native.available() and not native.available()


def test_op_wrappers_check_shapes_on_the_host():
    """Undersized or mistyped buffers are refused before any library call."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray

    def fake(shape, dtype=np.float32):
        return DeviceArray(shape, dtype, _ptr=0x10000, _owner=False)

    with pytest.raises(ValueError):
        ops.rmsnorm(fake((4, 8)), None, fake((4, 8)), 4, 16, 1e-6)
    with pytest.raises(ValueError):
        ops.act_mul("silu", fake(100), fake(99), fake(100))
    with pytest.raises(TypeError):
        ops.act_mul("silu", fake(100), fake(100, np.int32), fake(100))
    with pytest.raises(ValueError):
        ops.qk_norm_rope(fake((2, 4, 64)), 4, 2, 64, 64, k=fake((2, 1, 64)), n_k_heads=2)
    with pytest.raises(ValueError):
        ops.embed_gather(12, fake(1000, np.uint8), 10, 256, fake(4, np.int32), fake((4, 256)))
    with pytest.raises(ValueError):
        ops.embed_gather(12, fake(1440, np.uint8), 10, 250, fake(4, np.int32), fake((4, 250)))
    with pytest.raises(ValueError):
        ops.gated_rmsnorm_silu(fake((2, 64)), fake((2, 63)), fake(16), fake((2, 64)), 2, 64, 1e-6)


def test_reference_python_surface():
    """Names, parameters and defaults of engine/tensor_native.py:163-253,
    engine/transformer_native.py:25-229 and engine/native.py:22-229."""
    from aero_amd import native, tensor_native as TN, transformer_native as N

    def params(f):
        return [(p.name, p.default) for p in inspect.signature(f).parameters.values()]

    assert params(N.rope_tables) == [("head_dim", inspect._empty), ("positions", inspect._empty),
                                     ("base", inspect._empty), ("n_dims", None),
                                     ("freq_factors", None)]
    assert params(N.apply_rope) == [("x", inspect._empty), ("cos", inspect._empty),
                                    ("sin", inspect._empty), ("positions", None), ("mode", 0)]
    assert params(N.rmsnorm_rows) == [("x", inspect._empty), ("weight", None), ("eps", 1e-6)]
    assert params(N.l2norm_rows) == [("x", inspect._empty), ("weight", None), ("eps", 1e-6)]
    assert params(N.swiglu) == [("gate", inspect._empty), ("up", inspect._empty)]
    assert (N.ROPE_NEOX, N.ROPE_INTERLEAVED) == (0, 1)
    assert params(TN.rmsnorm) == [("x", inspect._empty), ("weight", inspect._empty),
                                  ("eps", inspect._empty)]
    assert params(TN.l2norm) == [("x", inspect._empty), ("weight", None), ("eps", 1e-6)]
    assert params(TN.rmsnorm_rows) == [("t", inspect._empty), ("eps", inspect._empty)]
    for f in (TN.silu, TN.gelu):
        assert params(f) == [("x", inspect._empty)]
    assert params(TN.mul) == [("a", inspect._empty), ("b", inspect._empty)]
    assert params(native.dequant) == [("dtype", inspect._empty), ("raw", inspect._empty),
                                      ("shape", inspect._empty), ("threads", 0)]
    assert params(native.matvec) == [("dtype", inspect._empty), ("w_bytes", inspect._empty),
                                     ("x", inspect._empty), ("threads", 1)]
    assert params(native.matmul) == [("dtype", inspect._empty), ("w_bytes", inspect._empty),
                                     ("X", inspect._empty), ("threads", 1)]
    assert (native.DTYPE_Q8_0, native.DTYPE_Q4_K, native.DTYPE_Q6_K) == (8, 12, 14)
    assert native.NATIVE_TYPES == {8, 12, 13, 14, 23}
    # input checks that run before the library is needed
    with pytest.raises(TypeError):
        TN._flat32(np.array(["a", "b"]))
    assert TN._flat32([1, 2]).dtype == np.float32
    with pytest.raises(TypeError):
        native._byte_view([1, 2])
    with pytest.raises(TypeError):
        native._byte_view(np.zeros(4, np.int32))
    assert native._byte_len(bytes(100)) == 100 and native._rows_in(bytes(288), 12, 256) == 2


def test_workload_bytes_match_the_published_roofline_table():
    """Algorithmic bytes of the Llama-3-8B 512-token shape (R=512, N=4096,
    H+HK=40, D=128, F=14336) per op."""
    from aero_amd import workloads as W
    assert W.bytes_rmsnorm(512, 4096) == 16_793_600
    assert W.bytes_rope(512, 40, 128, 128, False, True, False) == 20_971_520
    assert W.bytes_act(512, 14336) == 88_080_384
    assert W.bytes_embed(512, 4096, W.Q4_K) == 9_568_256 + 4 * 512
    assert W.bytes_gated(4096, 4096, 128) == 201_326_592 + 512


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "8"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_per_op_selector(monkeypatch):
    from aero_amd import select
    monkeypatch.setenv("AERO_GPU_OPS", "rmsnorm, rope")
    assert select.enabled("rmsnorm") and select.enabled("rope") and not select.enabled("act")
    assert select.enabled("act", override=True) and not select.enabled("rope", override=False)
    monkeypatch.setenv("AERO_GPU_OPS", "all")
    assert all(select.enabled(op) for op in select.OPS)
    monkeypatch.setenv("AERO_GPU_OPS", "none")
    assert not any(select.enabled(op) for op in select.OPS)
    monkeypatch.delenv("AERO_GPU_OPS")
    assert not select.enabled("embed")
    assert select.enabled("embed", default=True)        # a device-resident loop's default
    monkeypatch.setenv("AERO_GPU_OPS", "none")
    assert not select.enabled("embed", default=True)    # an explicit setting wins
    monkeypatch.setenv("AERO_GPU_OPS", "rmsnrom")
    with pytest.raises(ValueError):
        select.enabled("rmsnorm")
    with pytest.raises(ValueError):
        select.enabled("softmax")


def test_fusion_selector(monkeypatch):
    from aero_amd import select
    monkeypatch.delenv("AERO_GPU_FUSE", raising=False)
    assert all(select.fusion_enabled(f) for f in select.FUSIONS)
    monkeypatch.setenv("AERO_GPU_FUSE", "none")
    assert not any(select.fusion_enabled(f) for f in select.FUSIONS)
    assert select.fusion_enabled("act_gemm", override=True)
    monkeypatch.setenv("AERO_GPU_FUSE", "norm_gemm")
    assert select.fusion_enabled("norm_gemm") and not select.fusion_enabled("embed_norm")
    monkeypatch.setenv("AERO_GPU_FUSE", "norm_gem")
    with pytest.raises(ValueError):
        select.fusion_enabled("norm_gemm")
    with pytest.raises(ValueError):
        select.fusion_enabled("softmax")


def test_native_ssm_fallback_contract():
    """The reference's callers catch only SsmUnavailable and then run numpy
    (engine/ssm.py:215-221, :297-304; engine/moe.py:73-77). A head dim the GPU
    scan lacks (the reference's own tests use d = 6, tests/test_ssm_native.py:177)
    and the routines outside the path must raise exactly that, before any
    device work, so such a caller still gets its CPU result."""
    from aero_amd import native_ssm as NS
    from oracle import cpuref as O

    rng = np.random.default_rng(5)
    H, d = 3, 6
    q, k, v = (rng.standard_normal((H, d)).astype(np.float32) for _ in range(3))
    alpha, beta = rng.standard_normal(H).astype(np.float32), rng.standard_normal(H).astype(
        np.float32)
    a_log, dt_bias = rng.standard_normal(H).astype(np.float32) * 0.1, np.zeros(H, np.float32)
    state = rng.standard_normal((H, d, d)).astype(np.float32)

    def caller_step():                      # the shape of engine/ssm.py:215-221
        try:
            return NS.delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, 0.5)
        except NS.SsmUnavailable:
            return O.ssm_delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, 0.5)

    out, st = caller_step()
    want_out, want_st = O.ssm_delta_step(q, k, v, alpha, beta, a_log, dt_bias, state, 0.5)
    assert np.array_equal(out, want_out) and np.array_equal(st, want_st)
    T = 4
    qs = rng.standard_normal((T, H, d)).astype(np.float32)
    with pytest.raises(NS.SsmUnavailable, match="head dims"):
        NS.scan(qs, qs, qs, np.zeros((T, H), np.float32), np.zeros((T, H), np.float32),
                a_log, dt_bias, state, 0.5)
    for f in (NS.forward, NS.route, NS.expert_accum, NS.ffn_block):
        with pytest.raises(NS.SsmUnavailable):
            f()


def test_workspace_grows_only_and_plans_hold_what_they_recorded(monkeypatch):
    """Host logic of ops' scratch buffers, without a GPU: one buffer per op
    family, reallocated only when a call needs more (alternating 4096- and
    14336-column GEMMs keep the largest), and every buffer used while a plan
    records stays referenced by that plan after a larger call replaces it."""
    from aero_amd import device as D

    class FakeBuf:
        def __init__(self, shape, dtype=np.float32):
            self.nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize

    monkeypatch.setattr(D.DeviceArray, "empty", classmethod(lambda cls, s, dt=np.float32:
                                                            FakeBuf(s, dt)))
    ws = D.Workspace("split GEMM")
    small, big = 6 * 32 * 4096, 6 * 32 * 14336
    a = ws.get(small)
    b = ws.get(big)
    c = ws.get(small)
    assert b is c and a is not b and b.nbytes >= big
    assert ws.get(0) is None

    class FakePlan:
        def __init__(self):
            self._held = []
        hold = D.Plan.hold

    p = FakePlan()
    D._recording.plan = p
    try:
        r1 = ws.get(small)                  # the current (largest) buffer
        r2 = ws.get(2 * big)                # grows during recording
        ws.get(big)
    finally:
        D._recording.plan = None
    assert r1 is b and r2 is not b
    assert p._held == [b, r2]              # each once, in first-use order
    ws.get(4 * big)                         # outside the plan: replaces r2
    assert ws.buf is not r2 and p._held[1] is r2


def test_split_ok_follows_the_split_rule():
    """aero_hip_split_ok is host arithmetic over the split path's shape rule:
    Q4_K/Q5_K/Q8_0 rows of whole 16 bytes, Q6_K of whole 2048-value groups,
    IQ4_XS of whole 512, from a token count that depends on the matrix size."""
    from aero_amd import ops, workloads as W

    assert ops.split_ok(W.Q4_K, 4096, 6144, 512)
    assert ops.split_ok(W.Q5_K, 4096, 6144, 512)
    assert ops.split_ok(W.Q8_0, 4096, 6144, 512)
    assert ops.split_ok(W.Q6_K, 4096, 6144, 512)
    assert ops.split_ok(W.Q6_K, 14336, 4096, 512)
    assert ops.split_ok(W.IQ4_XS, 4096, 6144, 512)
    assert not ops.split_ok(W.Q6_K, 2560, 4096, 512)     # 2560 % 2048
    assert not ops.split_ok(W.Q8_0, 896, 1152, 512)      # 952-byte rows
    assert not ops.split_ok(W.F32, 4096, 4096, 512)
    assert not ops.split_ok(W.Q4_K, 4096, 6144, 2)       # below the token threshold
    assert ops.split_ok(W.Q4_K, 4096, 14336, 5) and not ops.split_ok(W.Q4_K, 4096, 14336, 4)
    assert not ops.split_ok(W.Q4_K, 4000, 4096, 512)     # not whole super-blocks


def test_attn_input_struct_layout(tmp_path):
    """aero_attn_input_t as the C compiler lays it out (gcc on the header)
    equals the ctypes mirror field for field: offsets and size."""
    fields = [f for f, _ in _lib.AttnInput._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "aero_hip.h"\n'
                   "int main(void) {\n"
                   + "".join(f'  printf("%zu\\n", offsetof(aero_attn_input_t, {f}));\n'
                             for f in fields)
                   + '  printf("%zu\\n", sizeof(aero_attn_input_t));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [getattr(_lib.AttnInput, f).offset for f in fields] + [ctypes_sizeof()]
    assert got == want


def ctypes_sizeof():
    import ctypes
    return ctypes.sizeof(_lib.AttnInput)
