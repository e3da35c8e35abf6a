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


def with_workspace(L, t, dw, dx, n_rows, n_cols, n_tok, partials=True):
    """aero_hip_matmul with a caller workspace: the split GEMM's own bytes and,
    with `partials`, room for its column splits' partials (the room the
    allocation-free entry has in its array)."""
    ws_bytes = L.aero_hip_matmul_workspace(t, n_cols, n_tok)
    assert ws_bytes > 0
    if partials:
        ws_bytes += L.aero_hip_split_partials_bytes(n_rows, n_cols, n_tok)
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
    # the larger call first, then smaller ones over the array it left behind;
    # 33 and 4 tokens split their columns (partials in the array too)
    for n_rows, n_cols, n_tok, seed in ((1024, 4096, 512, 1), (130, 2048, 33, 2),
                                        (4096, 14336, 4, 3)):
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


def test_few_tokens_without_partials_room_take_the_gemv(hip, oracle):
    """A few-token call given only the split GEMM's own workspace (no room for
    its column splits' partials) runs the GEMV rather than the unsplit split
    GEMM, which is slower there: bit-identical to the same call with no
    workspace at all."""
    L = _lib.lib()
    t, n_rows, n_cols, n_tok = W.Q4_K, 4096, 14336, 4
    assert L.aero_hip_split_partials_bytes(n_rows, n_cols, n_tok) > 0
    w, X = case(t, n_rows, n_cols, n_tok, 11)
    dw, dx = DA.from_numpy(w), DA.from_numpy(X)
    print(f"few-token split room rows={n_rows} cols={n_cols} tokens={n_tok}", flush=True)
    short = with_workspace(L, t, dw, dx, n_rows, n_cols, n_tok, partials=False)
    y = DA.empty((n_tok, n_rows))
    assert L.aero_hip_matmul(t, dw.ptr, dw.nbytes, dx.ptr, y.ptr, n_rows, n_cols, n_tok, None, 0,
                             None) == 1
    synchronize()
    assert bits_equal(short, y.numpy())
    assert rel_to_scale(short, oracle.matmul(t, w, X, n_rows)) <= RTOL


def test_overlapping_calls_on_two_streams_are_refused(hip):
    """A call on a second stream while the first stream's call may still be
    using the array is refused with a reason (not left to race); once the
    first stream is done, the second stream's call runs and gives the same
    bits. The first call is held behind ~2 ms of copies on its stream, so
    it is still queued when the second call is made."""
    from aero_amd import ops
    from aero_amd.device import Stream

    L = _lib.lib()
    t, n_rows, n_cols, n_tok = W.Q4_K, 1024, 4096, 64
    w, X = case(t, n_rows, n_cols, n_tok, 21)
    dw, dx = DA.from_numpy(w), DA.from_numpy(X)
    s1, s2 = Stream(), Stream()
    big = [(DA.empty(1 << 27), DA.empty(1 << 27)) for _ in range(2)]   # 2 x 512 MiB pairs
    y1, y2 = DA.empty((n_tok, n_rows)), DA.empty((n_tok, n_rows))
    print("noalloc overlap: copies then a call on stream 1, a call on stream 2", flush=True)
    for _ in range(4):
        for a, b in big:
            ops.copy_f32(a, b, stream=s1)
    assert L.aero_hip_matmul_noalloc(t, dw.ptr, dw.nbytes, dx.ptr, y1.ptr, n_rows, n_cols,
                                     n_tok, s1.handle) == 1, _lib.last_error()
    r = L.aero_hip_matmul_noalloc(t, dw.ptr, dw.nbytes, dx.ptr, y2.ptr, n_rows, n_cols, n_tok,
                                  s2.handle)
    assert r == 0 and "another stream" in _lib.last_error()
    s1.synchronize()
    assert L.aero_hip_matmul_noalloc(t, dw.ptr, dw.nbytes, dx.ptr, y2.ptr, n_rows, n_cols, n_tok,
                                     s2.handle) == 1, _lib.last_error()
    s2.synchronize()
    assert bits_equal(y1.numpy(), y2.numpy())
    s1.destroy()
    s2.destroy()
