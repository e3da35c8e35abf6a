"""GPU: the allocation-free matmul (aero_hip_matmul_noalloc, the split-x
GEMM with its workspace in a device array inside the library) against
aero_hip_matmul with a caller-allocated workspace, through the C-ABI.

The two run the same kernels on the same inputs, so their outputs must be
equal bit for bit. Two calls in a row, the second smaller, show that the
array's contents left by one call do not reach the next. The oracle's
matmul (the reference's src/kernels.cpp:520-538) is checked beside them to
the reference's RTOL.
"""
import numpy as np
import pytest

from conftest import RTOL, bits_equal, rel_to_scale
from aero_amd import _lib
from aero_amd import workloads as W
from aero_amd.device import DeviceArray as DA, synchronize

pytestmark = pytest.mark.gpu


def case(t, n_rows, n_cols, n_tok, seed):
    rng = np.random.default_rng(seed)
    w = W.make_table(t, n_rows * n_cols // 256, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    return w, X


def with_workspace(L, t, dw, dx, n_rows, n_cols, n_tok):
    ws_bytes = L.aero_hip_matmul_workspace(t, n_cols, n_tok)
    assert ws_bytes > 0
    ws = DA.empty((ws_bytes,), np.uint8)
    y = DA.empty((n_tok, n_rows))
    assert L.aero_hip_matmul(t, dw.ptr, dw.nbytes, dx.ptr, y.ptr, n_rows, n_cols, n_tok, ws.ptr,
                             ws_bytes, None) == 1, _lib.last_error()
    synchronize()
    return y.numpy()


def no_alloc(L, t, dw, dx, n_rows, n_cols, n_tok):
    y = DA.empty((n_tok, n_rows))
    assert L.aero_hip_matmul_noalloc(t, dw.ptr, dw.nbytes, dx.ptr, y.ptr, n_rows, n_cols, n_tok,
                                     None) == 1, _lib.last_error()
    synchronize()
    return y.numpy()


@pytest.mark.parametrize("t", [W.Q4_K, W.Q5_K])
def test_noalloc_matches_workspace_entry(hip, oracle, t):
    L = _lib.lib()
    assert L.aero_hip_matmul_noalloc_max_bytes() == 32 << 20
    # the larger call first, then a smaller one over the array it left behind
    for n_rows, n_cols, n_tok, seed in ((1024, 4096, 512, 1), (130, 2048, 33, 2)):
        print(f"noalloc type={t} rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
        assert L.aero_hip_matmul_workspace(t, n_cols, n_tok) <= 32 << 20
        w, X = case(t, n_rows, n_cols, n_tok, seed + t)
        dw, dx = DA.from_numpy(w), DA.from_numpy(X)
        got = no_alloc(L, t, dw, dx, n_rows, n_cols, n_tok)
        want = with_workspace(L, t, dw, dx, n_rows, n_cols, n_tok)
        assert bits_equal(got, want)
        assert rel_to_scale(got, oracle.matmul(t, w, X, n_rows)) <= RTOL


def test_noalloc_other_paths_and_refusal(hip, oracle):
    """Types and token counts without the split path need no scratch and run
    the same GEMV / fp32 GEMM as aero_hip_matmul; a call whose split
    workspace would exceed the array is refused on the host, before any
    launch, with the reason."""
    L = _lib.lib()
    for t, n_tok in ((W.Q6_K, 64), (W.Q4_K, 3)):
        w, X = case(t, 96, 512, n_tok, 7)
        dw, dx = DA.from_numpy(w), DA.from_numpy(X)
        got = no_alloc(L, t, dw, dx, 96, 512, n_tok)
        y = DA.empty((n_tok, 96))
        assert L.aero_hip_matmul(t, dw.ptr, dw.nbytes, dx.ptr, y.ptr, 96, 512, n_tok, None, 0,
                                 None) == 1
        synchronize()
        assert bits_equal(got, y.numpy())
        assert rel_to_scale(got, oracle.matmul(t, w, X, 96)) <= RTOL
    n_cols, n_tok = 14336, 1024
    assert L.aero_hip_matmul_workspace(W.Q4_K, n_cols, n_tok) > 32 << 20
    dx = DA.empty((n_tok, n_cols))
    dw = DA.empty((8 * (n_cols // 256) * 144,), np.uint8)
    y = DA.empty((n_tok, 8))
    assert L.aero_hip_matmul_noalloc(W.Q4_K, dw.ptr, dw.nbytes, dx.ptr, y.ptr, 8, n_cols, n_tok,
                                     None) == 0
    assert "scratch" in _lib.last_error()
