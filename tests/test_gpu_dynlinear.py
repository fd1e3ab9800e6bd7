"""GPU parity of lq_dynamic_linear_packed_f32 -- a dynamic int8 Linear at decode sizes in one
launch, with the layer norm (and residual add) before it folded in -- against the launches it
replaces, bit for bit: lq_(add_)layer_norm_f32, lq_dynamic_quantize_f32 on the unsigned grid
(codes c - 128) and lq_gemm_w8a8_packed (LQ_EPI_A_U8S8, float32 out, optional GELU).  The
product is also checked against its float64 definition from the integer sums."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

EPS_LN, EPS = np.float32(1e-5), np.float32(1e-8)


def _d(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


class _Weight:
    def __init__(self, L, rng, N, K):
        from lucid_amd import _C

        self.N, self.K = N, K
        self.codes = rng.integers(-127, 128, (N, K)).astype(np.int8)
        self.scale = rng.uniform(1e-3, 2e-2, N).astype(np.float32)
        self.bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
        self.d_codes, self.d_scale, self.d_bias = _d(L, self.codes), _d(L, self.scale), _d(L, self.bias)
        self.packed = L.empty((_C.lib().lq_packed_weights_size(N, K),), np.int8, "gpu")
        _C.call("lq_pack_weights_i8", self.d_codes.data_ptr(), K, N, K, self.packed.data_ptr(), None)
        self.sums = L.empty((N,), np.int32, "gpu")
        _C.call("lq_row_sums_i8", self.d_codes.data_ptr(), K, N, K, self.sums.data_ptr(), None)


def _sequence(L, w, x, res, src, gelu, qmin=0, qmax=255):
    """The separate launches: (sum, codes, qparams, y)."""
    from lucid_amd import _C

    M, K = x.shape
    dx = _d(L, x)
    a = dx
    if src != _C.DL_PLAIN:
        a = L.empty((M, K), np.float32, "gpu")
        if src == _C.DL_ADD_LN:
            _C.call("lq_add_layer_norm_f32", dx.data_ptr(), K, _d(L, res).data_ptr(), K, a.data_ptr(), K, M, K, None,
                    None, EPS_LN, None)
        else:
            _C.call("lq_layer_norm_f32", dx.data_ptr(), K, a.data_ptr(), K, M, K, None, None, EPS_LN, None)
    q = L.empty((M, K), np.int8, "gpu")
    qp = L.empty((4,), np.float32, "gpu")
    ws_n = max(_C.lib().lq_dynamic_quantize_workspace_size(M * K), 16)
    ws = L.empty((ws_n,), np.uint8, "gpu")
    _C.call("lq_dynamic_quantize_f32", a.data_ptr(), M * K, _C.U8S8, qmin, qmax, EPS, qp.data_ptr(), q.data_ptr(),
            ws.data_ptr(), ws_n, None)
    y = L.empty((M, w.N), np.float32, "gpu")
    g_n = max(_C.lib().lq_gemm_w8a8_workspace_size(M, w.N, K), 16)
    gws = L.empty((g_n,), np.uint8, "gpu")
    qa = qp.data_ptr()
    _C.call("lq_gemm_w8a8_packed", q.data_ptr(), K, w.packed.data_ptr(), y.data_ptr(), w.N, M, w.N, K, qa + 8, 0,
            w.d_scale.data_ptr(), 1, qa + 12, None, w.sums.data_ptr(), w.d_bias.data_ptr(), None, None, 0, 0,
            _C.OUT_F32, _C.EPI_A_U8S8 | (_C.EPI_GELU if gelu else 0), gws.data_ptr(), g_n, None)
    return dx.numpy(), q.numpy(), qp.numpy(), y.numpy()


def _one_launch(L, w, x, res, src, gelu, qmin=0, qmax=255):
    from lucid_amd import _C

    M, K = x.shape
    dx = _d(L, x)
    dres = _d(L, res) if res is not None else None
    s = L.empty((M, K), np.float32, "gpu") if src == _C.DL_ADD_LN else None
    qp = L.empty((4,), np.float32, "gpu")
    y = L.empty((M, w.N), np.float32, "gpu")
    _C.call("lq_dynamic_linear_packed_f32", dx.data_ptr(), K, dres.data_ptr() if dres is not None else None, K,
            s.data_ptr() if s is not None else None, K, src, None, None, EPS_LN, M, K, qmin, qmax, EPS,
            qp.data_ptr(), w.packed.data_ptr(), w.d_scale.data_ptr(), w.sums.data_ptr(), w.d_bias.data_ptr(), w.N,
            y.data_ptr(), w.N, _C.EPI_GELU if gelu else 0, None)
    return dx.numpy(), (s.numpy() if s is not None else None), qp.numpy(), y.numpy()


CASES = [  # (M, K, N, src, gelu): the decoder's four Linears and its head at batch 8, then edges
    (8, 512, 1536, "ADD_LN", False), (8, 512, 512, "PLAIN", False), (8, 512, 2048, "ADD_LN", True),
    (8, 2048, 512, "PLAIN", False), (8, 512, 32000, "ADD_LN", False), (1, 512, 1536, "LN", False),
    (16, 1024, 100, "PLAIN", True), (3, 64, 8200, "LN", False), (4, 2048, 8192, "ADD_LN", False),
    (2, 8192, 520, "PLAIN", False),
]


@pytest.mark.parametrize("M,K,N,src,gelu", CASES)
def test_one_launch_equals_the_launches(gpu, M, K, N, src, gelu):
    from lucid_amd import _C

    s = {"PLAIN": _C.DL_PLAIN, "LN": _C.DL_LN, "ADD_LN": _C.DL_ADD_LN}[src]
    rng = np.random.default_rng(M * 1000 + K + N)
    w = _Weight(gpu, rng, N, K)
    x = (rng.standard_normal((M, K)) * 2 + 0.5).astype(np.float32)
    res = rng.standard_normal((M, K)).astype(np.float32) if s == _C.DL_ADD_LN else None
    xs, q, qp, y = _sequence(gpu, w, x, res, s, gelu)
    x1, s1, qp1, y1 = _one_launch(gpu, w, x, res, s, gelu)
    np.testing.assert_array_equal(x1.view(np.uint32), x.view(np.uint32))  # x itself untouched
    if s == _C.DL_ADD_LN:  # the residual sum: the bits lq_add_layer_norm_f32 left in x
        np.testing.assert_array_equal(s1.view(np.uint32), xs.view(np.uint32))
    np.testing.assert_array_equal(qp1.view(np.uint32), qp.view(np.uint32))
    np.testing.assert_array_equal(y1.view(np.uint32), y.view(np.uint32))
    if not gelu:  # and the product from its definition: the exact integer sums in float64
        acc = (q.astype(np.int64) + 128 - int(qp[3])) @ w.codes.astype(np.int64).T
        want = acc * (np.float64(qp[2]) * w.scale.astype(np.float64)) + w.bias
        np.testing.assert_allclose(y1, want, rtol=2e-6, atol=1e-6 * np.abs(want).max())


def test_one_launch_grid_and_refusals(gpu):
    """A narrower grid (quint8 reduced range 0..127) gives the sequence's bits too; shapes past
    the one-launch limits and bad arguments are refused before any launch."""
    from lucid_amd import _C

    rng = np.random.default_rng(3)
    w = _Weight(gpu, rng, 64, 256)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    _, q, qp, y = _sequence(gpu, w, x, None, _C.DL_LN, False, 0, 127)
    _, _, qp1, y1 = _one_launch(gpu, w, x, None, _C.DL_LN, False, 0, 127)
    np.testing.assert_array_equal(qp1.view(np.uint32), qp.view(np.uint32))
    np.testing.assert_array_equal(y1.view(np.uint32), y.view(np.uint32))
    y = gpu.empty((17, 64), np.float32, "gpu")
    p = w.packed.data_ptr()
    base = dict(M=4, K=256, src=_C.DL_PLAIN, qmin=0, qmax=255, flags=0, res=None)

    def call(**kw):
        a = dict(base, **kw)
        _C.call("lq_dynamic_linear_packed_f32", y.data_ptr(), a["K"], a["res"], a["K"], None, a["K"], a["src"], None,
                None, EPS_LN, a["M"], a["K"], a["qmin"], a["qmax"], EPS, None, p, w.d_scale.data_ptr(),
                w.sums.data_ptr(), None, 64, y.data_ptr(), 64, a["flags"], None)

    for kw, msg in ((dict(M=17), "one-launch"), (dict(K=520), "one-launch"), (dict(M=16, K=2048), "one-launch"),
                    (dict(src=_C.DL_LN, M=8, K=2048), "one-launch"), (dict(src=7), "bad src"),
                    (dict(src=_C.DL_ADD_LN), "needs res"), (dict(qmin=-128, qmax=127), "unsigned"),
                    (dict(flags=_C.EPI_RELU), "flags")):
        with pytest.raises(_C.LucidError, match=msg):
            call(**kw)
