"""GPU parity of the quantized modules (nnq.Linear / LinearReLU / Quantize, nnqd.Linear) and
the prepare -> calibrate -> convert / quantize_dynamic pipelines.

Each module forward is checked twice:

* bit-exact against the oracle's integer composition of the same layer (weight observer ->
  qparams -> codes; activation codes; exact int32 sum; the documented epilogue);
* against Lucid's float composition (fake-quantize -> dequantized weight -> float GEMM ->
  fake-quantize, linear.py:206-215, dynamic/linear.py:85-92), evaluated in float64:
  fp32 outputs within rtol 1e-5 with atol = 1e-5 * max|expected| (the reference suite's
  assert_close_to_scale, lucid/test/_helpers/compare.py:54-86); requantized outputs at most
  one code apart, with the mismatch rate bounded.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import assert_close_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _reference_engine():
    """These tests cover the int8 sidecar layers: pin the engine that selects them (with the
    group-wise kernels present, "auto" routes group-divisible Linears to QuantizedLinearMLX)."""
    import lucid_amd.backends as backends

    backends.quantized.engine = "reference"
    yield
    backends.quantized.engine = "auto"


def _relu(y):
    return np.where(y <= 0, np.float32(0), y).astype(np.float32)


def _mlp_params(seed, dims=(784, 256, 10)):
    rng = np.random.default_rng(seed)
    ws, bs = [], []
    for i in range(len(dims) - 1):
        ws.append(rng.normal(0, 0.05, (dims[i + 1], dims[i])).astype(np.float32))
        bs.append(rng.normal(0, 0.05, dims[i + 1]).astype(np.float32))
    return rng, ws, bs


def _float_linear(L, W, b):
    import lucid_amd.nn as nn

    lin = nn.Linear(W.shape[1], W.shape[0])
    lin.weight = nn.Parameter(L.tensor(W))
    lin.bias = nn.Parameter(L.tensor(b))
    return lin


def _oracle_weight(W, qmin=-128, qmax=127):
    """Per-channel symmetric qint8 weight: observer -> qparams -> codes."""
    mn, mx = O.minmax_per_channel(W, 0)
    s, z = O.calc_qparams(mn, mx, True, True, qmin, qmax)
    q = O.quantize(W, O.recip_tensor(s), z, qmin, qmax, O.I8, ch_axis=0)
    return q, s, z


def _oracle_dynamic_linear(x, W, b):
    qw, sw, _ = _oracle_weight(W)
    r = O.minmax(x, mode=O.OBS_REPLACE)
    sx, zx = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    u = O.quantize(x, O.recip_tensor(sx), zx, 0, 255, O.U8S8)
    y = O.gemm_w8a8(u.reshape(-1, W.shape[1]), qw, sx, sw, za=float(zx) - 128.0, bias=b,
                    out_kind=O.OUT_F32)
    return y, (u, sx, zx, qw, sw)


def _lucid_dynamic_linear_f64(x, W, b):
    """Lucid's float composition in float64, and sum |terms| for a scale-aware tolerance."""
    qw, sw, zw = _oracle_weight(W)
    r = O.minmax(x, mode=O.OBS_REPLACE)
    sx, zx = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    xq, _ = O.fake_quantize(x, O.recip_tensor(sx), sx, zx, 0, 255)
    wd = O.dequantize(qw, O.I8, sw, zw, ch_axis=0)
    xd, wdd = xq.astype(np.float64), wd.astype(np.float64)
    return xd @ wdd.T + b


@pytest.mark.parametrize("M", [64, 1, 200])
def test_dynamic_mlp_config1(gpu, M):
    """Linear 784->256, ReLU, Linear 256->10, batch 64, quantize_dynamic."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.quantization import quantize_dynamic

    rng, (W1, W2), (b1, b2) = _mlp_params(2024)
    model = nn.Sequential(_float_linear(gpu, W1, b1), nn.ReLU(), _float_linear(gpu, W2, b2))
    qmodel = quantize_dynamic(model)
    assert isinstance(qmodel[0], nnqd.Linear) and isinstance(qmodel[2], nnqd.Linear)
    assert isinstance(model[0], nn.Linear)  # not in place
    x = rng.standard_normal((M, 784)).astype(np.float32)
    y = qmodel(gpu.tensor(x, device="gpu")).numpy()

    y1, _ = _oracle_dynamic_linear(x, W1, b1)
    h = _relu(y1)
    want, _ = _oracle_dynamic_linear(h, W2, b2)
    np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))

    # Lucid's float composition, layer by layer from the same inputs
    for xin, W, b, got in ((x, W1, b1, y1), (h, W2, b2, want)):
        ref = _lucid_dynamic_linear_f64(xin, W, b)
        assert_close_f32(got, ref)

    # weight buffers are Lucid's layout and values
    qw, sw, zw = _oracle_weight(W1)
    np.testing.assert_array_equal(qmodel[0].weight_int8.numpy(), qw)
    np.testing.assert_array_equal(qmodel[0].weight_scale.numpy(), sw)
    np.testing.assert_array_equal(qmodel[0].weight_zero_point.numpy(), zw)


def test_dynamic_linear_3d_input_and_no_bias(gpu):
    import lucid_amd.nn as nn
    from lucid_amd.quantization import quantize_dynamic

    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.05, (96, 128)).astype(np.float32)
    lin = nn.Linear(128, 96, bias=False)
    lin.weight = nn.Parameter(gpu.tensor(W))
    q = quantize_dynamic(nn.Sequential(lin))
    x = rng.standard_normal((2, 7, 128)).astype(np.float32)
    y = q(gpu.tensor(x, device="gpu")).numpy()
    assert y.shape == (2, 7, 96)
    want, _ = _oracle_dynamic_linear(x, W, None)
    np.testing.assert_array_equal(y.reshape(-1, 96).view(np.uint32), want.view(np.uint32))


def _static_model(L, W1, b1, W2, b2):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    return nn.Sequential(nnq.QuantStub(), _float_linear(L, W1, b1), nn.ReLU(),
                         _float_linear(L, W2, b2), nnq.DeQuantStub())


def _static_pipeline(L, seed=7, batches=4, M=64, dims=(784, 256, 10)):
    import lucid_amd.quantization as Q

    rng, (W1, W2), (b1, b2) = _mlp_params(seed, dims)
    model = _static_model(L, W1, b1, W2, b2)
    model = Q.fuse_modules(model, [["1", "2"]])
    prepared = Q.prepare(model, Q.get_minmax_qconfig())
    for _ in range(batches):
        prepared(L.tensor(rng.standard_normal((M, dims[0])).astype(np.float32), device="gpu"))
    return rng, Q.convert(prepared), (W1, b1, W2, b2)


@pytest.mark.parametrize("M", [64, 1, 300])
def test_static_ptq_linear_relu_exact(gpu, M):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    rng, q, (W1, b1, W2, b2) = _static_pipeline(gpu)
    assert [type(m) for m in q] == [nnq.Quantize, nnq.LinearReLU, nn.Identity, nnq.Linear,
                                    nnq.DeQuantize]
    x = rng.standard_normal((M, 784)).astype(np.float32)
    y = q(gpu.tensor(x, device="gpu"))
    assert y.is_code_backed
    got = y.numpy()

    s0, z0 = q[0].scale.numpy(), q[0].zero_point.numpy()
    c0 = O.quantize(x, O.recip_tensor(s0), z0, 0, 255, O.U8S8)
    layers = ((q[1], W1, b1, True), (q[3], W2, b2, False))
    codes, s_in, z_in = c0, s0, z0
    for mod, W, b, relu in layers:
        qw, sw, zw = _oracle_weight(W)
        np.testing.assert_array_equal(mod.weight_int8.numpy(), qw)
        np.testing.assert_array_equal(mod.weight_scale.numpy(), sw)
        S, Z = mod.scale.numpy(), mod.zero_point.numpy()
        codes = O.gemm_w8a8(codes, qw, s_in, sw, za=float(z_in) - 128.0, bias=b, out_scale=S,
                            out_zp=Z, qmin=0, qmax=255, out_kind=O.OUT_QU8S8, relu=relu)
        s_in, z_in = S, Z
    want = O.dequantize(codes, O.U8S8, s_in, z_in)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), codes)


def test_static_ptq_vs_float_composition(gpu):
    """One layer against Lucid's float composition from the same input codes: output codes
    at most one apart, mismatches (float GEMM rounding across a code boundary) rare."""
    rng, q, (W1, b1, _, _) = _static_pipeline(gpu)
    x = rng.standard_normal((256, 784)).astype(np.float32)
    s0, z0 = q[0].scale.numpy(), q[0].zero_point.numpy()
    c0 = O.quantize(x, O.recip_tensor(s0), z0, 0, 255, O.U8S8)
    h = q[1](q[0](gpu.tensor(x, device="gpu")))
    got = h.quant_source.codes.numpy().astype(np.int32)

    qw, sw, zw = _oracle_weight(W1)
    xd = O.dequantize(c0, O.U8S8, s0, z0).astype(np.float64)
    wd = O.dequantize(qw, O.I8, sw, zw, ch_axis=0).astype(np.float64)
    yf = np.maximum(xd @ wd.T + b1, 0.0).astype(np.float32)
    S, Z = q[1].scale.numpy(), q[1].zero_point.numpy()
    lit = O.quantize(yf, O.recip_tensor(S), Z, 0, 255, O.U8S8).astype(np.int32)
    diff = np.abs(got - lit)
    assert diff.max() <= 1
    assert np.mean(diff) < 5e-3, f"mismatch rate {np.mean(diff):.2e}"


def test_static_state_dict_round_trip(gpu):
    import lucid_amd.nn.quantized as nnq

    rng, q, _ = _static_pipeline(gpu)
    sd = q[1].state_dict()
    assert list(sd) == ["weight_int8", "weight_scale", "weight_zero_point", "bias", "scale",
                        "zero_point"]
    assert sd["weight_int8"].dtype == np.int8 and sd["scale"].shape == ()
    fresh = nnq.LinearReLU(784, 256)  # CPU buffers; loading copies values in
    fresh.load_state_dict(sd)
    x = gpu.tensor(rng.standard_normal((32, 784)).astype(np.float32), device="gpu")
    a = q[1](q[0](x)).numpy()
    b = fresh(q[0](x)).numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    # a later load replaces the cached device operands
    sd2 = {k: v for k, v in sd.items()}
    sd2["weight_int8"] = gpu.tensor(-sd["weight_int8"].numpy(), device="gpu")
    fresh.load_state_dict(sd2)
    c = fresh(q[0](x)).numpy()
    assert not np.array_equal(c, b)


def test_quantized_linear_float_input_literal_path(gpu):
    """A plain float input (not on a grid) takes Lucid's literal composition on the GPU."""
    rng, q, (W1, b1, _, _) = _static_pipeline(gpu)
    x = rng.standard_normal((16, 784)).astype(np.float32)
    y = q[1](gpu.tensor(x, device="gpu"))
    got = y.quant_source.codes.numpy().astype(np.int32)
    qw, sw, zw = _oracle_weight(W1)
    wd = O.dequantize(qw, O.I8, sw, zw, ch_axis=0).astype(np.float64)
    yf = np.maximum(x.astype(np.float64) @ wd.T + b1, 0.0).astype(np.float32)
    S, Z = q[1].scale.numpy(), q[1].zero_point.numpy()
    lit = O.quantize(yf, O.recip_tensor(S), Z, 0, 255, O.U8S8).astype(np.int32)
    assert np.abs(got - lit).max() <= 1


def test_uncalibrated_convert_warns(gpu):
    import lucid_amd.quantization as Q

    _, (W1, W2), (b1, b2) = _mlp_params(1, (64, 32, 8))
    model = _static_model(gpu, W1, b1, W2, b2)
    prepared = Q.prepare(model, Q.get_minmax_qconfig())
    with pytest.warns(UserWarning, match="never saw data"):
        Q.convert(prepared)


def test_qint8_output_grid(gpu):
    """A signed activation grid (qint8 observer) requantizes to int8 codes."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.quantization as Q
    from lucid_amd.quantization.observer import MinMaxObserver, PerChannelMinMaxObserver

    rng, (W1,), (b1,) = _mlp_params(11, (128, 64))
    model = nn.Sequential(nnq.QuantStub(), _float_linear(gpu, W1, b1), nnq.DeQuantStub())
    qc = Q.QConfig(activation=MinMaxObserver.with_args(qscheme=Q.per_tensor_symmetric,
                                                       qdtype=Q.qint8),
                   weight=PerChannelMinMaxObserver.with_args(ch_axis=0,
                                                             qscheme=Q.per_channel_symmetric,
                                                             qdtype=Q.qint8))
    prepared = Q.prepare(model, qc)
    prepared(gpu.tensor(rng.standard_normal((32, 128)).astype(np.float32), device="gpu"))
    q = Q.convert(prepared)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    y = q(gpu.tensor(x, device="gpu"))
    s0, z0 = q[0].scale.numpy(), q[0].zero_point.numpy()
    c0 = O.quantize(x, O.recip_tensor(s0), z0, -128, 127, O.I8)
    qw, sw, _ = _oracle_weight(W1)
    S, Z = q[1].scale.numpy(), q[1].zero_point.numpy()
    codes = O.gemm_w8a8(c0, qw, s0, sw, za=float(z0), bias=b1, out_scale=S, out_zp=Z,
                        qmin=-128, qmax=127, out_kind=O.OUT_Q8)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), codes)
    np.testing.assert_array_equal(y.numpy(), O.dequantize(codes, O.I8, S, Z))


# ------------------------------------------------------------------ convolution


def _conv_stack(L, rng):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    conv1 = nn.Conv2d(3, 16, 3, padding=1)
    bn = nn.BatchNorm2d(16)
    bn.running_mean = L.tensor(rng.normal(0, 0.1, 16).astype(np.float32))
    bn.running_var = L.tensor(rng.uniform(0.5, 1.5, 16).astype(np.float32))
    bn.weight = nn.Parameter(L.tensor(rng.normal(1, 0.1, 16).astype(np.float32)))
    bn.bias = nn.Parameter(L.tensor(rng.normal(0, 0.1, 16).astype(np.float32)))
    conv2 = nn.Conv2d(16, 32, 3, stride=2, padding=1)
    conv3 = nn.Conv2d(32, 24, 1, padding="same")
    conv4 = nn.Conv2d(24, 24, 3, padding=1, padding_mode="reflect", groups=4)
    return nn.Sequential(nnq.QuantStub(), conv1, bn, nn.ReLU(), conv2, nn.ReLU(), conv3, conv4,
                         nnq.DeQuantStub()).eval()


def _conv_pipeline(L, seed=3):
    import lucid_amd.quantization as Q

    rng = np.random.default_rng(seed)
    model = _conv_stack(L, rng)
    fused = Q.fuse_modules(model, [["1", "2", "3"], ["4", "5"]])
    prepared = Q.prepare(fused.to("gpu"), Q.get_minmax_qconfig())
    for _ in range(3):
        prepared(L.tensor(rng.standard_normal((4, 3, 16, 16)).astype(np.float32), device="gpu"))
    return rng, fused, Q.convert(prepared)


def test_static_conv_stack_exact(gpu):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from tests.test_gpu_conv import oracle_conv

    rng, fused, q = _conv_pipeline(gpu)
    assert [type(m) for m in q] == [nnq.Quantize, nnq.ConvReLU2d, nn.Identity, nn.Identity,
                                    nnq.ConvReLU2d, nn.Identity, nnq.Conv2d, nnq.Conv2d,
                                    nnq.DeQuantize]
    assert q[7].padding_mode == "reflect" and q[6].padding_str == "same"
    x = rng.standard_normal((2, 3, 16, 16)).astype(np.float32)
    y = q(gpu.tensor(x, device="gpu"))
    assert y.is_code_backed

    s0, z0 = q[0].scale.numpy(), q[0].zero_point.numpy()
    codes = O.quantize(x, O.recip_tensor(s0), z0, 0, 255, O.U8S8)
    s_in, z_in = s0, z0
    float_layers = (fused[1][0], fused[4][0], fused[6], fused[7])
    for mod, fl, relu, pad, mode in ((q[1], float_layers[0], True, (1, 1, 1, 1), 0),
                                     (q[4], float_layers[1], True, (1, 1, 1, 1), 0),
                                     (q[6], float_layers[2], False, (0, 0, 0, 0), 0),
                                     (q[7], float_layers[3], False, (1, 1, 1, 1), 1)):
        W = fl.weight.numpy()
        mn, mx = O.minmax_per_channel(W, 0)
        sw, zw = O.calc_qparams(mn, mx, True, True, -128, 127)
        qw = O.quantize(W, O.recip_tensor(sw), zw, -128, 127, O.I8, ch_axis=0)
        np.testing.assert_array_equal(mod.weight_int8.numpy(), qw)
        S, Z = mod.scale.numpy(), mod.zero_point.numpy()
        codes = oracle_conv(codes, qw, u8s8=True, za=float(z_in), stride=mod.stride, pad=pad,
                            dilation=mod.dilation, groups=mod.groups, mode=mode, a_scale=s_in,
                            w_scale=sw, bias=fl.bias.numpy(), out_kind=O.OUT_QU8S8,
                            out_scale=float(S), out_zp=float(Z), qmin=0, qmax=255, relu=relu)
        s_in, z_in = S, Z
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), codes)
    want = O.dequantize(codes, O.U8S8, s_in, z_in)
    np.testing.assert_array_equal(y.numpy().view(np.uint32), want.view(np.uint32))


def test_static_conv_vs_float_composition(gpu):
    """First conv against Lucid's float composition (dequantized kernel, float conv, ReLU,
    fake-quantize) from the same input codes: at most one code apart, rarely."""
    rng, fused, q = _conv_pipeline(gpu)
    x = rng.standard_normal((4, 3, 16, 16)).astype(np.float32)
    h = q[1](q[0](gpu.tensor(x, device="gpu")))
    got = h.quant_source.codes.numpy().astype(np.int32)
    s0, z0 = q[0].scale.numpy(), q[0].zero_point.numpy()
    c0 = O.quantize(x, O.recip_tensor(s0), z0, 0, 255, O.U8S8)
    xd = O.dequantize(c0, O.U8S8, s0, z0)
    W = q[1].weight_int8.numpy()
    wd = O.dequantize(W, O.I8, q[1].weight_scale.numpy(), q[1].weight_zero_point.numpy(), ch_axis=0)
    yf = O.conv2d_f32(xd, wd, q[1].bias.numpy(), pad=(1, 1, 1, 1))
    yf = np.where(yf <= 0, np.float32(0), yf).astype(np.float32)
    S, Z = q[1].scale.numpy(), q[1].zero_point.numpy()
    lit = O.quantize(yf, O.recip_tensor(S), Z, 0, 255, O.U8S8).astype(np.int32)
    diff = np.abs(got - lit)
    assert diff.max() <= 1 and diff.mean() < 5e-3


def test_conv_float_input_literal_path_and_state_dict(gpu):
    import lucid_amd.nn.quantized as nnq

    rng, fused, q = _conv_pipeline(gpu)
    x = rng.standard_normal((2, 16, 8, 8)).astype(np.float32)
    mod = q[4]
    y = mod(gpu.tensor(x, device="gpu"))  # plain float input: literal path
    W = mod.weight_int8.numpy()
    wd = O.dequantize(W, O.I8, mod.weight_scale.numpy(), mod.weight_zero_point.numpy(), ch_axis=0)
    yf = O.conv2d_f32(x, wd, mod.bias.numpy(), stride=(2, 2), pad=(1, 1, 1, 1))
    yf = np.where(yf <= 0, np.float32(0), yf).astype(np.float32)
    S, Z = mod.scale.numpy(), mod.zero_point.numpy()
    want = O.quantize(yf, O.recip_tensor(S), Z, 0, 255, O.U8S8)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)

    sd = mod.state_dict()
    assert list(sd) == ["weight_int8", "weight_scale", "weight_zero_point", "bias", "scale",
                        "zero_point"]
    fresh = nnq.ConvReLU2d(16, 32, 3, stride=2, padding=1)
    fresh.load_state_dict(sd)
    inp = q[0](gpu.tensor(rng.standard_normal((1, 3, 16, 16)).astype(np.float32), device="gpu"))
    h = q[1](inp)
    np.testing.assert_array_equal(fresh(h).numpy(), mod(h).numpy())


@pytest.mark.parametrize("M,N,K", [(2, 3, 4), (64, 256, 784), (64, 10, 256), (4096, 2048, 512),
                                   (8, 512, 2048), (8, 32000, 512), (33, 70, 129), (5, 6, 0)])
def test_float_linear_matches_oracle(gpu, M, N, K):
    """F.linear of the float model (lq_linear_f32) against the oracle's float64 x W^T + b at
    the configs' shapes (MLP, decoder projections and head), rtol 1e-5 scale-aware; an empty
    K leaves exactly the bias."""
    from lucid_amd.nn import functional as F

    rng = np.random.default_rng(M + N + K)
    x = rng.uniform(-1.0, 1.0, (M, K)).astype(np.float32)
    w = rng.normal(0, 0.05, (N, K)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    y = F.linear(gpu.tensor(x, device="gpu"), gpu.tensor(w, device="gpu"), gpu.tensor(b, device="gpu"))
    assert_close_f32(y.numpy(), O.linear(x, w, b))
    if K == 0:
        np.testing.assert_array_equal(y.numpy(), np.broadcast_to(b, (M, N)))


def test_float_linear_reference_golden(gpu):
    """The reference's own linear golden (lucid/test/numerical/golden/linear_2x4_4to3.npz,
    recipe test_golden.py:55-70) on the device, at that test's atol 1e-5."""
    import os

    from lucid_amd.nn import functional as F

    rng = np.random.default_rng(0)
    x = rng.uniform(-1.0, 1.0, size=(2, 4)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, size=(3, 4)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=(3,)).astype(np.float32)
    want = np.load(os.path.join(os.path.dirname(__file__), "golden", "lucid_linear_2x4_4to3.npz"))["out"]
    y = F.linear(gpu.tensor(x, device="gpu"), gpu.tensor(w, device="gpu"), gpu.tensor(b, device="gpu"))
    np.testing.assert_allclose(y.numpy(), want, atol=1e-5, rtol=0)
