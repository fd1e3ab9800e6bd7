"""The kernel instantiations the bench times, each checked bit-exactly against the oracle on
the shapes (or the path) the bench runs.

* W8A8 GEMM through the 256x256 LDS-DMA tile (the headline) and the 256x128 tile: every output
  kind with the full epilogue (per-row and per-column scales, bias, ReLU, activation and weight
  zero points) on shapes that reach each tile; the benched 4096^3 launches (int8 and f16 out)
  in full; the 4096x11008 shapes on sampled rows; the 128x128 tile at M = 1024.
* int8 Conv2d through the 256x64 tile: the ResNet-18 layers at batch 32 exactly as the bench
  configures them, plus every output kind on one 256x64 shape.
* Config 2: observer, qparams, quantize and dequantize over 2^24 and 2^28 elements with the
  0.1% x20 outliers, per tensor and per channel (C = 4096).

Each case asserts the kernel variant it reached (``lq_last_path``), so a change in the
dispatch thresholds cannot silently move a test off the instantiation it is meant to pin.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from test_gpu_conv import GRID as CONV_GRID
from test_gpu_conv import oracle_conv, run_conv
from test_gpu_gemm import GRID, KINDS, run_gemm

pytestmark = pytest.mark.gpu


def _codes(rng, shape, lo=-127, hi=127):
    return rng.integers(lo, hi + 1, size=shape, dtype=np.int64).astype(np.int8)


def _same_bits(got, want):
    if want.dtype == np.float16:
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    else:
        np.testing.assert_array_equal(np.ascontiguousarray(got).view(np.uint8),
                                      np.ascontiguousarray(want).view(np.uint8))


def _path():
    from lucid_amd import _C

    return _C.last_path()


# ------------------------------------------------------- GEMM 256x256 and 256x128


@pytest.mark.parametrize("M,N,K,path", [(2048, 4096, 256, "gemm dma 256x128"),
                                        (2100, 4100, 384, "gemm dma 256x128"),
                                        (4096, 4096, 256, "gemm dma 256x256"),
                                        (4000, 4050, 384, "gemm dma 256x256")])
def test_gemm_dma_every_kind_exact(gpu, M, N, K, path):
    """K % 128 == 0 with enough tiles for the DMA kernels: 256 tiles of 256x256 (one round)
    take the 256x256 kernel, fewer take 256 or more tiles of 256x128.  Every output kind, both
    epilogue forms (scales + bias; zero points + ReLU).  N = 4100 / 4050 leave 4- and 18-column
    tails handled by the scalar stores of the same kernel."""
    rng = np.random.default_rng(M + N + K)
    A = _codes(rng, (M, K), -128, 127)
    B = _codes(rng, (N, K))
    a_scale = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b_scale = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    zb = rng.integers(-3, 4, N).astype(np.float32)
    forms = ((None, None, True, False), (-5.0, zb, False, True))
    accs = [O.gemm_acc(A, B, 0 if za is None else int(za), None if zbv is None else zbv.astype(np.int32))
            for za, zbv, _, _ in forms]
    for kind in KINDS:
        qmin, qmax = GRID.get(kind, (-128, 127))
        out_scale, out_zp = 0.37, (128.0 if qmin == 0 else -3.0)
        for (za, zbv, with_bias, relu), acc in zip(forms, accs):
            print(f"gemm {path} M={M} N={N} K={K} kind={kind} za={za} relu={relu}", flush=True)
            got = run_gemm(gpu, A, B, kind, a_scale, b_scale, za, zbv, None,
                           bias if with_bias else None, out_scale, out_zp, qmin, qmax, relu)
            assert _path() == path
            want = O.gemm_epilogue(acc, a_scale, b_scale, bias if with_bias else None, out_scale,
                                   out_zp, qmin, qmax, kind, relu)
            _same_bits(got, want)


def _bench_gemm_args(M, N, K, seed):
    """The bench's synthetic headline inputs (bench.py Gemm): codes in [-127, 127], scales
    U[1e-3, 1e-1], bias N(0, 1), requantize with scale 64 and zero point 0."""
    rng = np.random.default_rng(seed)
    A = rng.integers(-127, 128, (M, K), dtype=np.int64).astype(np.int8)
    B = rng.integers(-127, 128, (N, K), dtype=np.int64).astype(np.int8)
    sa = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-1, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    return A, B, sa, sb, bias


def test_gemm_headline_4096_full_exact(gpu):
    """The benched launch (4096^3, fused requantize to int8; and f16 out), every output
    element against the oracle."""
    M = N = K = 4096
    A, B, sa, sb, bias = _bench_gemm_args(M, N, K, seed=0)
    acc = O.gemm_acc(A, B)
    for kind in (O.OUT_Q8, O.OUT_F16):
        print(f"gemm headline 4096^3 kind={kind}", flush=True)
        got = run_gemm(gpu, A, B, kind, sa, sb, bias=bias, out_scale=64.0, out_zp=0.0)
        assert _path() == "gemm dma 256x256"
        _same_bits(got, O.gemm_epilogue(acc, sa, sb, bias, 64.0, 0.0, -128, 127, kind, False))


@pytest.mark.parametrize("M,N,K,path", [(4096, 11008, 4096, "gemm dma 256x256"),
                                        (4096, 4096, 11008, "gemm dma 256x256"),
                                        (1024, 4096, 4096, "gemm dma 128x128 3-stage")])
def test_gemm_sweep_shapes_exact(gpu, M, N, K, path):
    """The sweep's large shapes: 64 sampled rows in full (4096-row shapes), every row at
    M = 1024; int8 and f16 outputs."""
    A, B, sa, sb, bias = _bench_gemm_args(M, N, K, seed=M + N + K)
    rng = np.random.default_rng(K)
    rows = np.arange(M) if M <= 1024 else np.sort(rng.choice(M, 64, replace=False))
    acc = O.gemm_acc(A[rows], B)
    for kind in (O.OUT_Q8, O.OUT_F16):
        print(f"gemm sweep M={M} N={N} K={K} kind={kind}", flush=True)
        got = run_gemm(gpu, A, B, kind, sa, sb, bias=bias, out_scale=64.0, out_zp=0.0)
        assert _path() == path
        _same_bits(got[rows], O.gemm_epilogue(acc, sa[rows], sb, bias, 64.0, 0.0, -128, 127, kind, False))


# ------------------------------------------------------------------- conv 256x64

RESNET18_B32 = (  # the bench's layers at batch 32: (name, Cin, Cout, H, k, stride, pad, kernel path)
    ("conv1 7x7/2", 3, 64, 224, 7, 2, 3, "conv taps dma 256x64"),
    ("layer1 3x3", 64, 64, 56, 3, 1, 1, "conv halo"),
    ("layer2 3x3/2", 64, 128, 56, 3, 2, 1, "conv dma 128x64"),
    ("layer2 3x3", 128, 128, 28, 3, 1, 1, "conv dma 128x64"),
    ("layer2 down 1x1/2", 64, 128, 56, 1, 2, 0, "conv dma 128x64"),
    ("layer3 3x3", 256, 256, 14, 3, 1, 1, "conv dma 128x64"),
    ("layer4 3x3", 512, 512, 7, 3, 1, 1, "conv dma 128x64 split-k"),
)


@pytest.mark.parametrize("layer", RESNET18_B32, ids=[r[0] for r in RESNET18_B32])
def test_conv_resnet18_batch32_exact(gpu, layer):
    """Each benched ResNet-18 layer at batch 32 as the bench configures it (unsigned
    activations kept as c - 128, zero point 128, per-channel weight scales, bias, ReLU,
    requantize to uint8): every output code against the oracle's convolution + epilogue."""
    name, cin, cout, H, k, st, pd, path = layer
    rng = np.random.default_rng(5 + cin + H)
    x = rng.integers(-128, 128, (32, cin, H, H)).astype(np.int8)
    w = rng.integers(-127, 128, (cout, cin, k, k)).astype(np.int8)
    kw = dict(u8s8=True, za=128.0, stride=(st, st), pad=(pd, pd, pd, pd), a_scale=0.02,
              w_scale=rng.uniform(1e-3, 1e-2, cout).astype(np.float32),
              bias=rng.standard_normal(cout).astype(np.float32), out_kind=O.OUT_QU8S8,
              out_scale=0.05, out_zp=0.0, qmin=0, qmax=255, relu=True)
    print(f"conv resnet18 b32 {name}", flush=True)
    got = run_conv(gpu, x, w, **kw)
    assert _path() == path
    _same_bits(got, oracle_conv(x, w, **kw))


@pytest.mark.parametrize("kind", [O.OUT_I32, O.OUT_F32, O.OUT_F16, O.OUT_Q8, O.OUT_QU8,
                                  O.OUT_FQ32, O.OUT_Q16, O.OUT_QU8S8])
def test_conv_256x64_every_kind_exact(gpu, kind):
    """N = 8, C = 64, 65 x 63, Cout = 128, 3 x 3 pad 1: 128 pixel tiles x 2 channel tiles
    = 256 tiles of 256x64, every output kind (a plane of 65 x 63, not a multiple of 16 bytes,
    keeps the integer kinds off the halo-staged kernel, which has its own tests)."""
    rng = np.random.default_rng(100 + kind)
    x = _codes(rng, (8, 64, 65, 63), -128, 127)
    w = _codes(rng, (128, 64, 3, 3))
    qmin, qmax = CONV_GRID.get(kind, (-128, 127))
    kw = dict(u8s8=True, za=120.0, stride=(1, 1), pad=(1, 1, 1, 1), out_kind=kind, qmin=qmin,
              qmax=qmax, out_zp=(128.0 if qmin == 0 else -2.0), relu=True,
              w_scale=rng.uniform(1e-3, 2e-2, 128).astype(np.float32),
              bias=rng.standard_normal(128).astype(np.float32))
    print(f"conv 256x64 kind={kind}", flush=True)
    got = run_conv(gpu, x, w, **kw)
    assert _path() == "conv dma 256x64"
    _same_bits(got, oracle_conv(x, w, **kw))


# ------------------------------------------------------- config 2 at full size


def _config2_data(n, seed):
    """N(0, 1) with 0.1% of the elements (uniformly chosen) multiplied by 20."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n, dtype=np.float32)
    idx = rng.choice(n, n // 1000, replace=False)
    x[idx] *= np.float32(20.0)
    return x


@pytest.mark.parametrize("log2n", [24, 28])
def test_config2_per_tensor_full_size(gpu, log2n):
    """MinMaxObserver -> calculate_qparams -> quantize -> dequantize (fp32 and fp16) over the
    whole tensor, per-tensor affine quint8 and symmetric qint8: every code and every float
    bit-exact; the observer's extrema equal numpy's."""
    Q = gpu.quantization
    n = 1 << log2n
    x = _config2_data(n, seed=log2n)
    xd = gpu.tensor(x, device="gpu")
    print(f"config2 per-tensor n=2^{log2n}", flush=True)
    obs = Q.MinMaxObserver(qscheme=Q.per_tensor_affine, qdtype=Q.quint8)
    obs(xd)
    mn, mx = float(obs.min_val.numpy()), float(obs.max_val.numpy())
    assert mn == float(x.min()) and mx == float(x.max())
    for qd, sym in ((Q.quint8, False), (Q.qint8, True)):
        s, z = O.calc_qparams(np.float32(mn), np.float32(mx), sym, qd.quant_min < 0, qd.quant_min,
                              qd.quant_max)
        code = O.I16 if qd.storage == "int16" else O.I8
        q = Q.quantize(xd, gpu.tensor(np.float32(s)), gpu.tensor(np.float32(z)), qd)
        want = O.quantize(x, O.recip_tensor(np.float32(s)), z, qd.quant_min, qd.quant_max, code)
        np.testing.assert_array_equal(q.numpy(), want)
        dq = Q.dequantize(q, gpu.tensor(np.float32(s)), gpu.tensor(np.float32(z))).numpy()
        np.testing.assert_array_equal(dq.view(np.uint32),
                                      O.dequantize(want, code, np.float32(s), z).view(np.uint32))
        del dq
        dh = Q.dequantize(q, gpu.tensor(np.float32(s)), gpu.tensor(np.float32(z)),
                          out_dtype=gpu.float16).numpy()
        np.testing.assert_array_equal(dh.view(np.uint16),
                                      O.dequantize(want, code, np.float32(s), z, y_dtype=O.F16)
                                      .view(np.uint16))
        del q, want, dh


@pytest.mark.parametrize("log2n", [24, 28])
def test_config2_per_channel_full_size(gpu, log2n):
    """PerChannelMinMaxObserver (C = 4096 leading) -> per-channel symmetric qint8 qparams ->
    quantize -> dequantize: every code and float bit-exact; per-channel extrema exact."""
    Q = gpu.quantization
    n = 1 << log2n
    x = _config2_data(n, seed=log2n + 1).reshape(4096, -1)
    xd = gpu.tensor(x, device="gpu")
    print(f"config2 per-channel n=2^{log2n}", flush=True)
    obs = Q.PerChannelMinMaxObserver(ch_axis=0, qscheme=Q.per_channel_symmetric, qdtype=Q.qint8)
    obs(xd)
    mn, mx = obs.min_val.numpy(), obs.max_val.numpy()
    np.testing.assert_array_equal(mn, x.min(axis=1))
    np.testing.assert_array_equal(mx, x.max(axis=1))
    s, z = O.calc_qparams(mn, mx, True, True, -128, 127)
    q = Q.quantize(xd, gpu.tensor(s), gpu.tensor(z), Q.qint8, ch_axis=0)
    want = O.quantize(x, O.recip_tensor(s), z, -128, 127, O.I8, ch_axis=0)
    np.testing.assert_array_equal(q.numpy(), want)
    dq = Q.dequantize(q, gpu.tensor(s), gpu.tensor(z), ch_axis=0).numpy()
    np.testing.assert_array_equal(dq.view(np.uint32),
                                  O.dequantize(want, O.I8, s, z, ch_axis=0).view(np.uint32))
