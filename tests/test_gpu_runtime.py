"""The runtime pieces around the kernels, on the GPU through the C ABI: stream-aware reuse of
freed device memory (``lq_record_stream`` / ``Tensor.record_stream``) and the lifetime of
captured graphs (``lq_graph_*``)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N = 4096


def _gemm_on(C, A, B, out, stream, reps):
    """`reps` int8 GEMMs of A [N, N] by B [N, N] into out (int32), queued on `stream`."""
    for _ in range(reps):
        C.call("lq_gemm_w8a8", A.data_ptr(), N, B.data_ptr(), N, out.data_ptr(), N, N, N, N, None, 0, None, 0,
               None, None, None, None, None, None, 0, 0, C.OUT_I32, 0, None, 0, stream)


def test_record_stream_holds_a_freed_block_until_the_side_stream_is_done(gpu):
    """A tensor read by work queued on a created stream and then dropped: without
    record_stream its block goes to the next null-stream allocation of that size at once;
    with it, not while that work is pending -- and the side-stream result is the one the
    original data gives."""
    from lucid_amd import _C

    rng = np.random.default_rng(0)
    a = rng.integers(-127, 128, (N, N)).astype(np.int8)
    b = rng.integers(-127, 128, (N, N)).astype(np.int8)
    st = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(st))
    try:
        # blocks earlier tests left in the cache would compete for the same size
        gpu.synchronize()
        _C.call("lq_empty_cache")
        B = gpu.tensor(b, device="gpu")
        out = gpu.empty((N, N), np.int32, "gpu")
        # without record_stream: immediate same-size reuse on the null stream
        A = gpu.tensor(a, device="gpu")
        gpu.synchronize()
        p = A.data_ptr()
        del A
        A2 = gpu.empty((N, N), np.int8, "gpu")
        assert A2.data_ptr() == p
        del A2
        # with record_stream: ~100 GEMMs (several ms) still queued on st when A is dropped
        A = gpu.tensor(a, device="gpu")
        gpu.synchronize()
        p = A.data_ptr()
        _gemm_on(_C, A, B, out, st, 100)
        A.record_stream(st)
        B.record_stream(st)
        out.record_stream(st)
        del A
        A2 = gpu.empty((N, N), np.int8, "gpu")
        assert A2.data_ptr() != p
        _C.call("lq_fill_u32", A2.data_ptr(), 0x01010101, N * N // 4, None)  # would clobber A's data
        _C.call("lq_stream_synchronize", st)
        got = out.numpy()
        rows = rng.choice(N, 16, replace=False)
        want = a[rows].astype(np.int64) @ b.astype(np.int64).T
        np.testing.assert_array_equal(got[rows], want)
        # after the side stream is done, A's block is free for the null stream again
        A3 = gpu.empty((N, N), np.int8, "gpu")
        assert A3.data_ptr() == p
    finally:
        _C.call("lq_stream_synchronize", st)
        _C.call("lq_stream_destroy", st)


def test_record_stream_rejects_foreign_pointers(gpu):
    from lucid_amd import _C

    x = np.zeros(16, np.uint8)
    assert _C.lib().lq_record_stream(ctypes.c_void_p(x.ctypes.data), None) == -1
    assert b"not from lq_malloc" in _C.lib().lq_last_error()


def test_graph_handle_replays_and_destroys(gpu):
    """A captured fill replayed three times, with eager work between replays, then the
    handle destroyed (the captured graph and its executable form go together)."""
    from lucid_amd import _C

    st = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(st))
    y = gpu.empty((1 << 20,), np.uint32, "gpu")
    try:
        _C.call("lq_graph_begin_capture", st)
        _C.call("lq_fill_u32", y.data_ptr(), 7, 1 << 20, st)
        exe = ctypes.c_void_p()
        _C.call("lq_graph_end_capture", st, ctypes.byref(exe))
        for _ in range(3):
            _C.call("lq_fill_u32", y.data_ptr(), 0, 1 << 20, None)
            gpu.synchronize()
            _C.call("lq_graph_launch", exe, st)
            _C.call("lq_stream_synchronize", st)
            assert (y.numpy() == 7).all()
        _C.call("lq_graph_destroy", exe)
        assert _C.lib().lq_graph_destroy(None) == 0
    finally:
        _C.call("lq_stream_destroy", st)
