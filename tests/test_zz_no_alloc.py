"""lq_gemm_w8a8_noalloc (workspace in the library's static per-GPU scratch array) against
lq_gemm_w8a8 with a caller workspace, through the C ABI: bit-exact on two calls in a row, the
second smaller, on paths that use the scratch (activation and weight code sums, split-K
partial sums and counters), with another call in between that fills the scratch with
different sums; and the size limit refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _dev(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


def _run(L, fn, A, B, kind, sa, sb, za, zb, bias, out_scale, out_zp, relu):
    """One call of lq_gemm_w8a8 (fn == "ws") or lq_gemm_w8a8_noalloc (fn == "noalloc")."""
    from lucid_amd import _C

    M, K = A.shape
    N = B.shape[0]
    dt = {O.OUT_Q8: np.int8, O.OUT_F32: np.float32, O.OUT_I32: np.int32, O.OUT_F16: np.float16}[kind]
    dA, dB = _dev(L, A), _dev(L, B)
    dC = L.empty((M, N), dt, "gpu")
    keep = []

    def opt(v):
        if v is None:
            return None
        t = _dev(L, np.atleast_1d(np.asarray(v, np.float32)))
        keep.append(t)
        return t.data_ptr()

    args = [dA.data_ptr(), K, dB.data_ptr(), K, dC.data_ptr(), N, M, N, K, opt(sa), 1, opt(sb), 1,
            opt(za), opt(zb), None, opt(bias), opt(out_scale), opt(out_zp), -128, 127, kind,
            _C.EPI_RELU if relu else 0]
    if fn == "ws":
        ws_bytes = _C.lib().lq_gemm_w8a8_workspace_size(M, N, K)
        ws = L.empty((max(ws_bytes, 1),), np.uint8, "gpu")
        _C.call("lq_gemm_w8a8", *args, ws.data_ptr(), ws_bytes, None)
    else:
        _C.call("lq_gemm_w8a8_noalloc", *args, None)
    path = _C.last_path()
    return dC.numpy(), path


def _case(rng, M, N, K, with_zb):
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    zb = rng.integers(-3, 4, N).astype(np.float32) if with_zb else None
    return A, B, sa, sb, float(rng.integers(-9, 10)), zb, bias


@pytest.mark.parametrize("kind", [O.OUT_Q8, O.OUT_F32])
def test_noalloc_matches_workspace_entry_point(gpu, kind):
    rng = np.random.default_rng(77 + kind)
    # 1: split-K 128x128 tiles (few tiles, long K), activation and weight zero points:
    #    code sums and split partials / counters all in the scratch
    # 2: a smaller call right after (activation zero point only, skinny kernel)
    # 3: the first shape again after a different-sized use of the scratch
    shapes = [(200, 1024, 4096, True, "gemm 128x128 split-k"), (48, 520, 1024, False, "gemm skinny"),
              (200, 1024, 4096, True, "gemm 128x128 split-k")]
    for M, N, K, with_zb, path in shapes:
        A, B, sa, sb, za, zb, bias = _case(rng, M, N, K, with_zb)
        print(f"noalloc M={M} N={N} K={K} kind={kind}", flush=True)
        want, p_ws = _run(gpu, "ws", A, B, kind, sa, sb, za, zb, bias, 0.5, -2.0, True)
        got, p_na = _run(gpu, "noalloc", A, B, kind, sa, sb, za, zb, bias, 0.5, -2.0, True)
        assert p_ws == p_na == path
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
        ref = O.gemm_w8a8(A, B, sa, sb, za=za, zb=zb, bias=bias, out_scale=0.5, out_zp=-2.0,
                          qmin=-128, qmax=127, out_kind=kind, relu=True)
        np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8))


def test_noalloc_refuses_shapes_beyond_its_scratch(gpu):
    from lucid_amd import _C

    lib = _C.lib()
    cap = lib.lq_gemm_w8a8_noalloc_scratch_bytes()
    assert cap == 16 << 20
    for M, N, K in ((1, 1 << 22, 64), (32640, 128, 128)):  # weight code sums; split-K partials
        assert lib.lq_gemm_w8a8_workspace_size(M, N, K) > cap
        rc = lib.lq_gemm_w8a8_noalloc(None, K, None, K, None, N, M, N, K, None, 0, None, 0, None,
                                      None, None, None, None, None, -128, 127, O.OUT_I32, 0, None)
        assert rc == -3  # LQ_ERR_UNSUPPORTED, before any launch
        assert b"scratch" in lib.lq_last_error()
