"""GPU parity of the weight-only kernels (lucid_amd/csrc/lq_wo.hip) through the C ABI.

* ``lq_gemv_w8`` (per-channel int8 weight, float activations): against the oracle's
  float64 ``x @ dequantize(W)^T + bias``.  fp32 outputs within rtol 1e-5 and fp16 outputs
  within rtol 1e-3, each with atol = rtol * max|expected| (the reference suite's
  ``assert_close_to_scale``, lucid/test/_helpers/compare.py:54-86).
* group-wise ``quantize`` / ``dequantize``: bit-exact against the oracle's restatement of
  the documented formula (lucid/quantization/_qgemm.py:84-97, 167-170);
* ``quantized_matmul``: against float64 ``x @ w_hat^T`` at the reference bench's parity
  gate (max error / max |y| <= 1e-4, tools/bench_quantized_dispatch.py) and the scale-aware
  1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import BF16_RTOL, F16_RTOL, assert_close_f16, assert_close_f32, assert_close_to_scale

pytestmark = pytest.mark.gpu


def _t(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


def _close(got, ref, half=False):
    """fp32 outputs within rtol 1e-5, fp16 within 1e-3, both with atol = rtol * max|ref|."""
    (assert_close_f16 if half else assert_close_f32)(got, ref)


def run_gemv(L, x, W, s, z=None, b=None, relu=False, half=False, ldw=None):
    from lucid_amd import _C

    M, K = x.shape
    N = W.shape[0]
    ldw = ldw or K
    Wp = np.zeros((N, ldw), np.int8)
    Wp[:, :K] = W
    xd = _t(L, x.astype(np.float16 if half else np.float32))
    dW, ds = _t(L, Wp), _t(L, s.astype(np.float32))
    dz = _t(L, z.astype(np.float32)) if z is not None else None
    db = _t(L, b.astype(np.float32)) if b is not None else None
    y = L.empty((M, N), np.float16 if half else np.float32, "gpu")
    ws_bytes = _C.lib().lq_gemv_w8_workspace_size(M, N, K)
    ws = L.empty((max(ws_bytes, 1),), np.uint8, "gpu")
    _C.call("lq_gemv_w8", xd.data_ptr(), _C.F16 if half else _C.F32, K, dW.data_ptr(), ldw,
            ds.data_ptr(), dz.data_ptr() if dz is not None else None,
            db.data_ptr() if db is not None else None, y.data_ptr(), N, M, N, K,
            _C.EPI_RELU if relu else 0, ws.data_ptr(), ws_bytes, None)
    return y.numpy()


def _gemv_ref(x, W, s, z=None, b=None, relu=False):
    """The oracle's dequantize -> linear (float64 accumulation)."""
    return O.gemv_w8(x, W, s, w_zp=z, bias=b, relu=relu)


GEMV_SHAPES = [(1, 4096, 4096), (16, 4096, 4096), (1, 11008, 4096), (8, 4096, 11008),
               (2, 96, 784), (17, 256, 784), (33, 100, 1000), (64, 10, 256), (100, 300, 512),
               (1, 1, 16), (5, 70, 48)]


@pytest.mark.parametrize("M,N,K", GEMV_SHAPES)
def test_gemv_w8_fp32(gpu, M, N, K):
    rng = np.random.default_rng(M * 131 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, ::97] *= 20.0  # outliers
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    got = run_gemv(gpu, x, W, s, b=b)
    ref = _gemv_ref(x, W, s, b=b)
    _close(got, ref)


@pytest.mark.parametrize("K", [4096, 1008])
def test_gemv_w8_row_loop_is_bit_identical(gpu, K):
    """One activation row with per-channel weights runs a persistent grid: a wave takes rows
    gw, gw + S, ... (S = every wave of the grid).  Row r's arithmetic must not depend on which
    wave or which pass takes it: the rows of an 11008-row call equal, bit for bit, the same rows
    computed in calls over 4096-row slices (one row per wave) and over a 1000-row slice
    (K = 1008: one 16-byte chunk per lane)."""
    rng = np.random.default_rng(K + 7)
    x = rng.standard_normal((1, K)).astype(np.float32)
    W = rng.integers(-128, 128, (11008, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, 11008).astype(np.float32)
    b = rng.standard_normal(11008).astype(np.float32)
    full = run_gemv(gpu, x, W, s, b=b, relu=True)
    for lo, hi in ((0, 4096), (4096, 8192), (8192, 11008), (5000, 6000)):
        part = run_gemv(gpu, x, W[lo:hi], s[lo:hi], b=b[lo:hi], relu=True)
        np.testing.assert_array_equal(full[:, lo:hi].view(np.uint32), part.view(np.uint32))
    _close(full, _gemv_ref(x, W, s, b=b, relu=True))


@pytest.mark.parametrize("M,N,K", [(4, 256, 784), (16, 1024, 4096), (1, 64, 1000)])
def test_gemv_w8_zero_point_relu_and_ldw(gpu, M, N, K):
    rng = np.random.default_rng(7 + M)
    x = (rng.standard_normal((M, K)) * 1e3).astype(np.float32)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    z = rng.integers(-5, 6, N).astype(np.float32)
    ref = _gemv_ref(x, W, s, z=z, relu=True)
    _close(run_gemv(gpu, x, W, s, z=z, relu=True), ref)
    _close(run_gemv(gpu, x, W, s, z=z, relu=True, ldw=K + 48), ref)  # 16-aligned rows
    _close(run_gemv(gpu, x, W, s, z=z, relu=True, ldw=K + 3), ref)   # unaligned rows


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (16, 1024, 1024), (3, 50, 784)])
def test_gemv_w8_fp16(gpu, M, N, K):
    rng = np.random.default_rng(11 + M)
    x = rng.standard_normal((M, K)).astype(np.float16)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    got = run_gemv(gpu, x.astype(np.float32), W, s, b=b, half=True)
    ref = _gemv_ref(x.astype(np.float32), W, s, b=b)
    _close(got, ref, half=True)


@pytest.mark.parametrize("M,N,K", [(17, 64, 256), (24, 4096, 4096), (37, 300, 784), (19, 50, 1000)])
def test_gemv_w8_presplit_matches_inline(gpu, M, N, K):
    """Above 16 rows, with a workspace the fp32 activations are split into fp16 halves once
    per call; the products and their order are those of the split done inside every
    workgroup, so both calls agree bit for bit (with rows of very different magnitude to
    exercise the per-block pre-scale)."""
    from lucid_amd import _C

    rng = np.random.default_rng(M * 7 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e-20
    x[-1] *= 1e20
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    z = rng.integers(-3, 4, N).astype(np.float32)
    ws_bytes = _C.lib().lq_gemv_w8_workspace_size(M, N, K)
    assert ws_bytes > 0
    xd, dW, ds, dz = _t(gpu, x), _t(gpu, W), _t(gpu, s), _t(gpu, z)
    outs = []
    for wsb in (ws_bytes, 0):
        ws = gpu.empty((max(wsb, 1),), np.uint8, "gpu")
        y = gpu.empty((M, N), np.float32, "gpu")
        _C.call("lq_gemv_w8", xd.data_ptr(), _C.F32, K, dW.data_ptr(), K, ds.data_ptr(), dz.data_ptr(), None,
                y.data_ptr(), N, M, N, K, 0, ws.data_ptr() if wsb else None, wsb, None)
        outs.append(y.numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    ref = _gemv_ref(x, W, s, z=z)
    _close(outs[0], ref)


SPLIT_K_SHAPES = [(16, 4096, 4096), (3, 4608, 4096), (7, 11008, 4096), (16, 4096, 11008), (12, 100, 784),
                  (16, 1000, 1024), (13, 64, 2048), (14, 300, 16)]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,N,K", SPLIT_K_SHAPES)
def test_gemv_w8_split_k(gpu, M, N, K, half):
    """3 <= M <= 16 with the workspace, from 12 rows or over 16 MB of weight: the split-K
    kernel (x split once per workgroup into LDS, the K ranges' sums added in range order by a
    second launch).  Against the oracle at
    the same tolerance, with a zero point, bias and ReLU; three calls in a row give the same
    bits."""
    from lucid_amd import _C

    print(f"gemv split-k M={M} N={N} K={K} half={half}", flush=True)
    rng = np.random.default_rng(M * 1000 + K + half)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, ::53] *= 30.0
    x[-1] *= 1e-6
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2 if half else 1e-1, N).astype(np.float32)
    z = rng.integers(-4, 5, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    outs = [run_gemv(gpu, x, W, s, z=z, b=b, relu=True, half=half) for _ in range(3)]
    assert _C.last_path() in ("wo split-k", "wo split-k single range")
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint16 if half else np.uint32),
                                      outs[0].view(np.uint16 if half else np.uint32))
    xr = x.astype(np.float16).astype(np.float32) if half else x
    _close(outs[0], _gemv_ref(xr, W, s, z=z, b=b, relu=True), half=half)


def test_gemv_w8_split_k_interleaved_shapes(gpu):
    """Calls of different shapes sharing one workspace, alternating: each call's result
    depends only on its own operands (same bits on every repetition)."""
    from lucid_amd import _C

    rng = np.random.default_rng(5)
    cases = []
    for (M, N, K) in ((16, 4096, 4096), (12, 256, 3072), (16, 11008, 4096)):
        x = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.integers(-128, 128, (N, K)).astype(np.int8)
        s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
        cases.append((x, W, s, _gemv_ref(x, W, s)))
    nbytes = max(_C.lib().lq_gemv_w8_workspace_size(c[0].shape[0], c[1].shape[0], c[0].shape[1]) for c in cases)
    ws = gpu.empty((nbytes,), np.uint8, "gpu")
    first = {}
    for rep in range(3):
        for i, (x, W, s, ref) in enumerate(cases):
            M, K = x.shape
            N = W.shape[0]
            y = gpu.empty((M, N), np.float32, "gpu")
            _C.call("lq_gemv_w8", _t(gpu, x).data_ptr(), _C.F32, K, _t(gpu, W).data_ptr(), K,
                    _t(gpu, s).data_ptr(), None, None, y.data_ptr(), N, M, N, K, 0, ws.data_ptr(), nbytes, None)
            got = y.numpy()
            if rep == 0:
                _close(got, ref)
                first[i] = got
            else:
                np.testing.assert_array_equal(got, first[i])


def run_gemv_packed(L, x, W, s, z=None, b=None, relu=False, half=False):
    from lucid_amd import _C

    M, K = x.shape
    N = W.shape[0]
    dW = _t(L, W)
    pk = L.empty((max(_C.lib().lq_packed_weights_size(N, K), 16),), np.int8, "gpu")
    _C.call("lq_pack_weights_i8", dW.data_ptr(), K, N, K, pk.data_ptr(), None)
    xd = _t(L, x.astype(np.float16 if half else np.float32))
    ds = _t(L, s.astype(np.float32))
    dz = _t(L, z.astype(np.float32)) if z is not None else None
    db = _t(L, b.astype(np.float32)) if b is not None else None
    y = L.empty((M, N), np.float16 if half else np.float32, "gpu")
    ws_bytes = _C.lib().lq_gemv_w8_packed_workspace_size(M, N, K)
    ws = L.empty((max(ws_bytes, 1),), np.uint8, "gpu")
    _C.call("lq_gemv_w8_packed", xd.data_ptr(), _C.F16 if half else _C.F32, K, pk.data_ptr(), ds.data_ptr(),
            dz.data_ptr() if dz is not None else None, db.data_ptr() if db is not None else None, y.data_ptr(),
            N, M, N, K, _C.EPI_RELU if relu else 0, ws.data_ptr(), ws_bytes, None)
    return y.numpy()


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,N,K", [(16, 4096, 4096), (1, 11008, 4096), (2, 4096, 11008), (8, 100, 784),
                                   (3, 1000, 1024), (16, 70, 16), (5, 33, 528)])
def test_gemv_w8_packed(gpu, M, N, K, half):
    """The decode entry over the MFMA-packed weight: against the oracle like lq_gemv_w8, with a
    zero point, bias and ReLU, and bit for bit lq_gemv_w8 where that takes its split-K route
    (same kernel, same products and order; only where the weight bytes come from differs)."""
    from lucid_amd import _C

    print(f"gemv packed M={M} N={N} K={K} half={half}", flush=True)
    rng = np.random.default_rng(M * 31 + N + K + half)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, ::41] *= 25.0
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2 if half else 1e-1, N).astype(np.float32)
    z = rng.integers(-4, 5, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    got = run_gemv_packed(gpu, x, W, s, z=z, b=b, relu=True, half=half)
    assert _C.last_path() in ("wo packed split-k", "wo packed split-k single range")
    xr = x.astype(np.float16).astype(np.float32) if half else x
    _close(got, _gemv_ref(xr, W, s, z=z, b=b, relu=True), half=half)
    rowmajor = run_gemv(gpu, x, W, s, z=z, b=b, relu=True, half=half)
    if _C.last_path() in ("wo split-k", "wo split-k single range"):
        np.testing.assert_array_equal(got.view(np.uint16 if half else np.uint32),
                                      rowmajor.view(np.uint16 if half else np.uint32))


def test_gemv_w8_packed_rejects(gpu):
    from lucid_amd import _C

    with pytest.raises(_C.LucidError, match="16 activation rows"):
        _C.call("lq_gemv_w8_packed", 16, _C.F32, 64, 16, 16, None, None, 16, 64, 17, 64, 64, 0, None, 0, None)
    with pytest.raises(_C.LucidError, match="multiple of 16"):
        _C.call("lq_gemv_w8_packed", 16, _C.F32, 72, 16, 16, None, None, 16, 64, 4, 64, 72, 0, None, 0, None)


def test_gemv_w8_tiny_and_huge_rows(gpu):
    """Per-row pre-scaling: rows of very different magnitude in one call."""
    rng = np.random.default_rng(3)
    M, N, K = 4, 128, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e-30
    x[1] *= 1e30
    x[2] = 0.0
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    got = run_gemv(gpu, x, W, s)
    ref = _gemv_ref(x, W, s)
    _close(got, ref)
    assert np.all(got[2] == 0.0)


# ----------------------------------------------------------------- group-wise


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_group_quantize_dequantize_exact(gpu, bits, gs):
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(bits * 1000 + gs)
    N, K = 96, 1024
    w = rng.standard_normal((N, K)).astype(np.float32)
    w[3, :gs] = 0.25  # a constant group
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    op, os_, ob = O.group_quantize(w, gs, bits)
    assert packed.dtype == np.int32 and packed.shape == (N, K * bits // 32)
    np.testing.assert_array_equal(packed.numpy().view(np.uint32), op)
    np.testing.assert_array_equal(scales.numpy(), os_)
    np.testing.assert_array_equal(biases.numpy(), ob)
    dense = _qgemm.dequantize(packed, scales, biases, group_size=gs, bits=bits)
    want = O.group_dequantize(op, os_, ob, gs, bits)
    np.testing.assert_array_equal(dense.numpy().view(np.uint32), want.view(np.uint32))
    nob = _qgemm.dequantize(packed, scales, None, group_size=gs, bits=bits)
    np.testing.assert_array_equal(nob.numpy(), O.group_dequantize(op, os_, None, gs, bits))
    # half-step reconstruction bound (lucid/quantization/_qgemm.py dequantize docstring)
    err = np.abs(want - w).reshape(N, K // gs, gs)
    assert np.all(err <= os_[:, :, None] * 0.5 + 1e-6)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 2, 8, 32, 70])
def test_quantized_matmul_parity(gpu, bits, gs, M):
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(bits + gs + M)
    N, K = 1024, 1024
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    y = _qgemm.quantized_matmul(_t(gpu, x), packed, scales, biases, transpose=True,
                                group_size=gs, bits=bits).numpy()
    wd = O.group_dequantize(packed.numpy().view(np.uint32), scales.numpy(), biases.numpy(), gs,
                            bits).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    assert np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-12) <= 1e-4
    _close(y, ref)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_group_matmul_presplit_matches_inline(gpu, bits, gs):
    """The once-per-call activation split (workspace given) against the in-workgroup split
    (no workspace): bit for bit."""
    from lucid_amd import _C
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(bits * 3 + gs)
    M, N, K = 19, 200, 1024
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[1] *= 1e-15
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    ws_bytes = _C.lib().lq_group_matmul_workspace_size(M, N, K, gs)
    assert ws_bytes > 0
    xd = _t(gpu, x)
    outs = []
    for wsb in (ws_bytes, 0):
        ws = gpu.empty((max(wsb, 1),), np.uint8, "gpu")
        y = gpu.empty((M, N), np.float32, "gpu")
        _C.call("lq_group_matmul", xd.data_ptr(), _C.F32, K, packed.data_ptr(), scales.data_ptr(),
                biases.data_ptr(), None, y.data_ptr(), N, M, N, K, gs, bits, 1, 0,
                ws.data_ptr() if wsb else None, wsb, None)
        outs.append(y.numpy())
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", [(16, 4096, 4096), (5, 4608, 4096), (12, 1000, 2048)])
def test_group_matmul_split_k(gpu, M, N, K, bits, gs):
    """Group-wise weights on the split-K kernel (3 <= M <= 16 with the workspace): the bench
    gate and the scale-aware 1e-5 against float64, repeatable bit for bit."""
    from lucid_amd import _C
    from lucid_amd.quantization import _qgemm

    print(f"group split-k M={M} N={N} K={K} bits={bits} gs={gs}", flush=True)
    rng = np.random.default_rng(M + N + bits + gs)
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    ws_bytes = _C.lib().lq_group_matmul_workspace_size(M, N, K, gs)
    ws = gpu.empty((max(ws_bytes, 1),), np.uint8, "gpu")
    xd, bd = _t(gpu, x), _t(gpu, b)
    outs = []
    for _ in range(2):
        y = gpu.empty((M, N), np.float32, "gpu")
        _C.call("lq_group_matmul", xd.data_ptr(), _C.F32, K, packed.data_ptr(), scales.data_ptr(),
                biases.data_ptr(), bd.data_ptr(), y.data_ptr(), N, M, N, K, gs, bits, 1, 0, ws.data_ptr(), ws_bytes,
                None)
        outs.append(y.numpy())
        assert _C.last_path() in ("wo split-k", "wo split-k single range")
    np.testing.assert_array_equal(outs[0], outs[1])
    wd = O.group_dequantize(packed.numpy().view(np.uint32), scales.numpy(), biases.numpy(), gs,
                            bits).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T + b
    assert np.max(np.abs(outs[0] - ref)) / max(np.max(np.abs(ref)), 1e-12) <= 1e-4
    _close(outs[0], ref)


@pytest.mark.parametrize("M,N,K,bits,gs", [(1, 4096, 4096, 4, 64), (16, 11008, 4096, 8, 64),
                                           (8, 4096, 11008, 4, 128), (3, 100, 192, 8, 32)])
def test_quantized_matmul_shapes_bias_relu_fp16(gpu, M, N, K, bits, gs):
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(M + N)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    wd = O.group_dequantize(packed.numpy().view(np.uint32), scales.numpy(), biases.numpy(), gs,
                            bits).astype(np.float64)
    for half in (False, True):
        xin = x.astype(np.float16) if half else x
        y = _qgemm.quantized_matmul(_t(gpu, xin), packed, scales, biases, group_size=gs,
                                    bits=bits, bias=_t(gpu, b), relu=True)
        assert y.dtype == (np.float16 if half else np.float32)
        xd = xin.astype(np.float64)
        if half:  # scales, group biases and bias in half, the product rounded to half
            ref = O.group_matmul(xd, packed.numpy().view(np.uint32), scales.numpy(), biases.numpy(), gs,
                                 bits, "f16", bias=b, relu=True)
        else:
            ref = np.maximum(xd @ wd.T + b, 0.0)
        _close(y.numpy(), ref, half=half)


def _ulp(v, dt):
    """Spacing of the half / bfloat16 values at |v| (their normal range)."""
    a = np.maximum(np.abs(v), 2.0 ** -14 if dt == "f16" else 2.0 ** -126)
    return np.ldexp(1.0, np.floor(np.log2(a)).astype(int) - (10 if dt == "f16" else 7))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("M,N,K,bits,gs,transpose", [(1, 4096, 4096, 4, 64, True), (2, 1024, 1024, 8, 32, True),
                                                     (5, 4608, 4096, 4, 64, True), (16, 4096, 4096, 4, 64, True),
                                                     (40, 512, 1024, 8, 128, True), (24, 300, 256, 4, 64, False)])
def test_quantized_matmul_half_dtype_rule(gpu, dt, M, N, K, bits, gs, transpose):
    """Lucid's dtype rule for half / bfloat16 activations (QuantizedMatmul.cpp:153-164,
    mlx_linear.py:215-222): scales, group biases and bias cast to x's dtype, the product in
    that dtype, the bias added there.  Compared in the type's own bits with the oracle's
    float64 composition rounded once: >= 97% of the outputs identical, the rest within one ulp
    (of the product before the bias) plus the float32 sum's tolerance, where the kernel's
    float32 sum lies near a rounding boundary.  The same outputs against the
    composition that keeps float32 scales (the cast left out) match visibly less often, so the
    test separates the two."""
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(M * 7 + N + bits)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    d_in, d_out = (K, N) if transpose else (N, K)
    x32 = rng.standard_normal((M, d_in)).astype(np.float32)
    b = rng.standard_normal(d_out).astype(np.float32)
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    if dt == "f16":
        xh = x32.astype(np.float16)
        xval = xh.astype(np.float64)
    else:
        xh = gpu.bf16_from_f32(x32)
        xval = O.bf16_round(x32).astype(np.float64)
        np.testing.assert_array_equal(gpu.bf16_to_f32(xh), O.bf16_round(x32))
    y = _qgemm.quantized_matmul(_t(gpu, xh), packed, scales, biases, transpose=transpose, group_size=gs,
                                bits=bits, bias=_t(gpu, b))
    assert y.dtype == xh.dtype and y.shape == (M, d_out)
    got = y.numpy()
    got = got.astype(np.float64) if dt == "f16" else gpu.bf16_to_f32(got).astype(np.float64)
    p, s, bb = packed.numpy().view(np.uint32), scales.numpy(), biases.numpy()
    want = O.group_matmul(xval, p, s, bb, gs, bits, dt, bias=b, transpose=transpose)
    no_cast = O.round_to(O.round_to(O.group_matmul(xval, p, s, bb, gs, bits, "f32", transpose=transpose), dt) +
                         O.round_to(b, dt), dt)
    assert np.isfinite(got).all()
    same = float(np.mean(got == want))
    same_no_cast = float(np.mean(got == no_cast))
    # a one-ulp step of the product before the bias is many ulps of a sum that cancels, and
    # where the product itself cancels, the float32 sum's own error (1e-5 of the largest
    # product, the fp32 tolerance) can exceed half an ulp of the small result
    pre = O.group_matmul(xval, p, s, bb, gs, bits, dt, transpose=transpose)
    mag = np.maximum(np.maximum(np.abs(got), np.abs(want)), np.abs(pre))
    err = np.maximum(np.abs(got - want) - 1e-5 * np.max(np.abs(pre)), 0.0)
    worst = float(np.max(err / _ulp(mag, dt)))
    print(f"{dt} M={M} N={N} K={K}: identical {same:.4f} (without the cast {same_no_cast:.4f}), worst {worst} ulp")
    assert same >= 0.97 and worst <= 1.0
    assert same_no_cast < same - 0.03
    assert_close_to_scale(got, want, F16_RTOL if dt == "f16" else BF16_RTOL, floor=2.0 ** -24)


def test_quantized_linear_mlx_module(gpu):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    rng = np.random.default_rng(0)
    lin = nn.Linear(256, 64)
    lin.weight = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, (64, 256)).astype(np.float32)))
    lin.bias = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, 64).astype(np.float32)))
    q = nnq.QuantizedLinearMLX.from_float(lin, bits=4, group_size=64, relu=True)
    sd = q.state_dict()
    assert list(sd) == ["packed_weight", "scales", "biases", "bias"]
    assert sd["packed_weight"].dtype == np.int32 and sd["packed_weight"].shape == (64, 32)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    y_gpu = q(gpu.tensor(x, device="gpu"))
    y_cpu = q(gpu.tensor(x))  # device-transparent: host in, host out
    assert y_cpu.device == "cpu" and y_gpu.device == "gpu"
    np.testing.assert_array_equal(y_cpu.numpy(), y_gpu.numpy())
    p, s, bb = O.group_quantize(lin.weight.numpy(), 64, 4)
    wd = O.group_dequantize(p, s, bb, 64, 4).astype(np.float64)
    ref = np.maximum(x.astype(np.float64) @ wd.T + lin.bias.numpy(), 0.0)
    _close(y_gpu.numpy(), ref)
    fresh = nnq.QuantizedLinearMLX(256, 64, bits=4, group_size=64, relu=True)
    fresh.load_state_dict(sd)
    np.testing.assert_array_equal(fresh(gpu.tensor(x, device="gpu")).numpy(), y_gpu.numpy())


def test_engine_routes_linear_family(gpu):
    """auto / mlx_group route Linear layers whose in_features a group size divides to the
    group-wise layer; 'reference' keeps the int8 sidecar layers (_quantize.py:134-185)."""
    import lucid_amd.backends as backends
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.quantization import quantize_dynamic

    assert backends.quantized.available
    model = nn.Sequential(nn.Linear(784, 256), nn.ReLU(), nn.Linear(256, 10)).to("gpu")
    q = backends.quantized
    try:
        for engine in ("auto", "mlx_group"):
            q.engine = engine
            m = quantize_dynamic(model)
            assert isinstance(m[0], nnqd.Linear)            # 784 divides by no group size
            assert isinstance(m[2], nnq.QuantizedLinearMLX) and m[2].group_size == 64
            assert m[2].bits == 8
        q.engine = "reference"
        m = quantize_dynamic(model)
        assert isinstance(m[2], nnqd.Linear)
    finally:
        q.engine = "auto"


def test_dispatch_bench_harness(gpu):
    """The bench_quantized_dispatch counterpart: parity gate, three paths, reference keys."""
    from lucid_amd import bench_quantized_dispatch as bqd

    rep = bqd.run(iters=2, width=256)
    rows = rep["rows"]
    assert len(rows) == 2 * 4 * 3
    assert {r["path"] for r in rows} == {"packed", "cached_dense", "dequant_each_call"}
    for r in rows:
        assert r["parity_relative_error"] <= 1e-4
        assert r["p5_ms"] <= r["median_ms"] <= r["p95_ms"]
        for key in ("bits", "m", "n", "k", "first_ms", "GB/s", "hbm_roofline_frac", "TOPS"):
            assert key in r


# ------------------------------------------- transpose=False and the QLoRA input gradient


def _packed_case(gpu, rng, N, K, gs, bits, scale=0.05):
    from lucid_amd.quantization import _qgemm

    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    packed, scales, biases = _qgemm.quantize(_t(gpu, w), group_size=gs, bits=bits)
    wd = O.group_dequantize(packed.numpy().view(np.uint32), scales.numpy(), biases.numpy(), gs,
                            bits).astype(np.float64)
    return packed, scales, biases, wd


@pytest.mark.parametrize("M,N,K,bits,gs", [(1, 64, 64, 8, 64), (70, 200, 96, 4, 32),
                                           (33, 1000, 384, 8, 128), (128, 512, 1024, 4, 64),
                                           (5, 7, 4096, 8, 64)])
def test_quantized_matmul_no_transpose(gpu, M, N, K, bits, gs):
    """``x @ w_hat`` (x [M, N] -> [M, K]) with bias / ReLU and fp16 inputs, against float64."""
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(M * 7 + N)
    packed, scales, biases, wd = _packed_case(gpu, rng, N, K, gs, bits)
    x = rng.standard_normal((M, N)).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    y = _qgemm.quantized_matmul(_t(gpu, x), packed, scales, biases, transpose=False, group_size=gs,
                                bits=bits)
    assert y.shape == (M, K) and y.dtype == np.float32
    ref = x.astype(np.float64) @ wd
    _close(y.numpy(), ref)
    for half in (False, True):
        xin = x.astype(np.float16) if half else x
        y = _qgemm.quantized_matmul(_t(gpu, xin), packed, scales, biases, transpose=False,
                                    group_size=gs, bits=bits, bias=_t(gpu, b), relu=True)
        assert y.dtype == (np.float16 if half else np.float32)
        xd = xin.astype(np.float64)
        _close(y.numpy(), np.maximum(xd @ wd + b, 0.0), half=half)


def test_quantized_matmul_no_transpose_without_group_biases_and_batched(gpu):
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(5)
    packed, scales, _, _ = _packed_case(gpu, rng, 48, 256, 64, 4)
    wd = O.group_dequantize(packed.numpy().view(np.uint32), scales.numpy(), None, 64, 4).astype(np.float64)
    x = rng.standard_normal((2, 3, 48)).astype(np.float32)
    y = _qgemm.quantized_matmul(_t(gpu, x), packed, scales, None, transpose=False, group_size=64, bits=4)
    assert y.shape == (2, 3, 256)
    xd = x.astype(np.float64)
    _close(y.numpy(), xd @ wd)


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_matmul_backward_is_the_adjoint(gpu, transpose, bits):
    """QLoRA's dX (QuantizedMatmulBackward::apply, QuantizedMatmul.cpp:73-90): against float64
    ``dY dequant(W)`` (or its transpose), and the adjoint identity
    ``<dY, f(x)> = <dX(dY), x>`` of the linear map f -- a transposed or mis-grouped product
    fails it."""
    from lucid_amd.quantization import _qgemm

    rng = np.random.default_rng(bits + 10 * transpose)
    M, N, K, gs = 37, 160, 512, 64
    packed, scales, biases, wd = _packed_case(gpu, rng, N, K, gs, bits)
    d_in, d_out = (K, N) if transpose else (N, K)
    x = rng.standard_normal((M, d_in)).astype(np.float32)
    dy = rng.standard_normal((M, d_out)).astype(np.float32)
    y = _qgemm.quantized_matmul(_t(gpu, x), packed, scales, biases, transpose=transpose, group_size=gs,
                                bits=bits).numpy().astype(np.float64)
    dx = _qgemm.quantized_matmul_backward(_t(gpu, dy), packed, scales, biases, transpose=transpose,
                                          group_size=gs, bits=bits)
    assert dx.shape == x.shape and dx.dtype == np.float32
    dyd = dy.astype(np.float64)
    wmat = wd if transpose else wd.T   # dX = dY @ w_deq (swapaxes when transpose=False)
    _close(dx.numpy(), dyd @ wmat)
    lhs = float(np.sum(dyd * y))
    rhs = float(np.sum(dx.numpy().astype(np.float64) * x))
    mag = float(np.abs(dyd).ravel() @ (np.abs(x.astype(np.float64)) @ np.abs(wd.T if transpose else wd)).ravel())
    assert abs(lhs - rhs) <= 1e-5 * mag


def test_group_matmul_no_transpose_empty_reduction(gpu):
    """N = 0: x [M, 0] @ w_hat[0, K] is the bias alone."""
    from lucid_amd import _C

    M, K = 3, 64
    b = np.arange(K, dtype=np.float32) - 30
    bd = _t(gpu, b)
    x = gpu.empty((M, 1), np.float32, "gpu")
    y = gpu.empty((M, K), np.float32, "gpu")
    _C.call("lq_group_matmul", x.data_ptr(), _C.F32, 0, None, None, None, bd.data_ptr(), y.data_ptr(), K,
            M, 0, K, 64, 8, 0, _C.EPI_RELU, None, 0, None)
    np.testing.assert_array_equal(y.numpy(), np.broadcast_to(np.maximum(b, 0), (M, K)))


def test_quantized_linear_mlx_module_bf16(gpu):
    """QuantizedLinearMLX on bfloat16 activations (host and device): bfloat16 out, the dtype
    rule of the reference (bias cast and added in bfloat16, then ReLU)."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    rng = np.random.default_rng(4)
    lin = nn.Linear(512, 96)
    lin.weight = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, (96, 512)).astype(np.float32)))
    lin.bias = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, 96).astype(np.float32)))
    q = nnq.QuantizedLinearMLX.from_float(lin, bits=4, group_size=64, relu=True)
    x = gpu.bf16_from_f32(rng.standard_normal((6, 512)).astype(np.float32))
    y_gpu = q(gpu.tensor(x, device="gpu"))
    y_cpu = q(gpu.tensor(x))
    assert y_gpu.dtype == gpu.bfloat16 and y_cpu.device == "cpu"
    np.testing.assert_array_equal(y_cpu.numpy().view(np.uint16), y_gpu.numpy().view(np.uint16))
    sd = q.state_dict()
    want = O.group_matmul(gpu.bf16_to_f32(x), sd["packed_weight"].numpy().view(np.uint32), sd["scales"].numpy(),
                          sd["biases"].numpy(), 64, 4, "bf16", bias=lin.bias.numpy(), relu=True)
    got = gpu.bf16_to_f32(y_gpu.numpy()).astype(np.float64)
    assert np.mean(got == want) >= 0.97
    pre = O.group_matmul(gpu.bf16_to_f32(x), sd["packed_weight"].numpy().view(np.uint32), sd["scales"].numpy(),
                         sd["biases"].numpy(), 64, 4, "bf16")
    mag = np.maximum(np.maximum(np.abs(got), np.abs(want)), np.abs(pre))
    assert np.max(np.abs(got - want) / _ulp(mag, "bf16")) <= 1.0

