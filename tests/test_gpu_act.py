"""GPU parity of the activations (lq_qact; nn.Sigmoid / Tanh / Hardswish / Hardsigmoid / ELU /
LeakyReLU and their quantized counterparts in nn.quantized) against the oracle.

* hardswish / hardsigmoid / leaky_relu are IEEE add / divide / multiply / compare chains:
  bit-exact float outputs and codes;
* sigmoid / tanh / elu go through exp / tanh, whose last bit is the math library's (Lucid's
  is vForce's): float outputs within a few float32 ulps of the oracle, and the output codes
  equal to the grid codes of the GPU's own float result (the quantize stage is bit-exact);
* inputs as float32 or as the codes of a code-backed activation; NaN, infinities, -0, the
  hardsigmoid knots at -3 / 3; misaligned pointers and ragged lengths (scalar path);
* the flow of the reference's own tests (lucid/test/unit/quantization/
  test_module_breadth.py:53-89): Linear + activation, default qconfig, calibrate, convert.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

EXACT = (O.ACT_HARDSWISH, O.ACT_HARDSIGMOID, O.ACT_LEAKY_RELU)
ULPS = {O.ACT_SIGMOID: 4, O.ACT_TANH: 3, O.ACT_ELU: 4}
PARAM = {O.ACT_ELU: 1.5, O.ACT_LEAKY_RELU: 0.2}
NAMES = {O.ACT_SIGMOID: "sigmoid", O.ACT_TANH: "tanh", O.ACT_HARDSWISH: "hardswish",
         O.ACT_HARDSIGMOID: "hardsigmoid", O.ACT_ELU: "elu", O.ACT_LEAKY_RELU: "leaky_relu"}


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    special = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, -3.0, 3.0, -2.9999998, 2.9999998, 90.0, -90.0,
                        1e-30, -1e-30], np.float32)
    k = min(n, special.size)
    x[:k] = special[:k]
    return x


def _ulps(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    both_nan = np.isnan(a) & np.isnan(b)
    same = (a == b) | both_nan
    u = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32)).astype(np.float64)
    with np.errstate(invalid="ignore"):
        d = np.where(same, 0.0, np.abs(a - b) / u)
    return np.where(np.isnan(d), np.inf, d)


def _check_float(op, got, want):
    if op in EXACT:
        # bit-exact, except a NaN's sign / payload (hardswish(-inf) = -inf * 0 is the host
        # CPU's default NaN on one side, the GPU's on the other)
        nan = np.isnan(want)
        np.testing.assert_array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    else:
        u = _ulps(got, want)
        if op == O.ACT_ELU:
            # exp(x) - 1 cancels near 0: an ulp of exp's result near 1 (2^-24 .. 2^-23) is the
            # error unit there, times alpha, rather than an ulp of the small result
            with np.errstate(invalid="ignore"):
                slack = np.abs(got.astype(np.float64) - want) <= 2 * PARAM[op] * 2.0 ** -23
            u = np.where(slack, 0.0, u)
        assert u.max() <= ULPS[op], f"{NAMES[op]}: {u.max()} ulps at x index {int(np.argmax(u))}"


def _qact(gpu, op, x_ptr, x_type, xs, xz, n, y_ptr, out_type, s=None, z=None, qmin=0, qmax=0):
    from lucid_amd import _C

    _C.call("lq_qact", op, x_ptr, x_type, xs, xz, n, float(np.float32(PARAM.get(op, 0.0))),
            s.data_ptr() if s is not None else None, z.data_ptr() if z is not None else None, qmin, qmax,
            out_type, y_ptr, None)


@pytest.mark.parametrize("op", list(NAMES))
@pytest.mark.parametrize("n", [1, 15, 4096 + 13, (1 << 20) + 3])
def test_float_activation_matches_oracle(gpu, op, n):
    from lucid_amd import _C

    x = _inputs(n, op * 10 + n % 7)
    xd = gpu.tensor(x, device="gpu")
    y = gpu.empty((n,), np.float32, "gpu")
    _qact(gpu, op, xd.data_ptr(), _C.F32, None, None, n, y.data_ptr(), _C.F32)
    _check_float(op, y.numpy(), O.activation(x, op, PARAM.get(op, 0.0)))


@pytest.mark.parametrize("op", list(NAMES))
def test_misaligned_pointers(gpu, op):
    # one element past a 16-byte boundary on both sides: the one-element-per-step path
    from lucid_amd import _C

    n = 3001
    x = _inputs(n + 1, op)
    xd = gpu.tensor(x, device="gpu")
    y = gpu.empty((n + 1,), np.float32, "gpu")
    _qact(gpu, op, xd.data_ptr() + 4, _C.F32, None, None, n, y.data_ptr() + 4, _C.F32)
    got = y.numpy()[1:]
    _check_float(op, got, O.activation(x[1:], op, PARAM.get(op, 0.0)))


@pytest.mark.parametrize("op", list(NAMES))
@pytest.mark.parametrize("in_kind", ["f32", "i8", "u8s8"])
@pytest.mark.parametrize("out_grid", [(O.U8S8, 0, 255, 0.011, 97.0), (O.I8, -128, 127, 0.013, 0.0),
                                      (O.U8, 0, 255, 0.02, 13.0), (O.I16, -1000, 1000, 0.004, 5.0)])
def test_quantized_activation_codes(gpu, op, in_kind, out_grid):
    from lucid_amd import _C

    code, qmin, qmax, s_out, z_out = out_grid
    n = 70001
    x = _inputs(n, op + len(in_kind))
    if in_kind == "f32":
        xin, xtype, sx, zx, val = x, _C.F32, None, None, x
    else:
        xtype = O.I8 if in_kind == "i8" else O.U8S8
        s_in = np.float32(0.05)
        z_in = np.float32(0.0 if in_kind == "i8" else 120.0)
        lo, hi = (-128, 127) if in_kind == "i8" else (0, 255)
        xin = O.quantize(x, O.recip_tensor(np.array([s_in]))[0], z_in, lo, hi, xtype)
        val = O.dequantize(xin, xtype, s_in, z_in)
        sx, zx = gpu.tensor(np.array([s_in]), device="gpu"), gpu.tensor(np.array([z_in]), device="gpu")
    xd = gpu.tensor(np.ascontiguousarray(xin), device="gpu")
    so, zo = gpu.tensor(np.array([s_out], np.float32), device="gpu"), gpu.tensor(np.array([z_out], np.float32),
                                                                                device="gpu")
    ct = {O.U8S8: np.int8, O.I8: np.int8, O.U8: np.uint8, O.I16: np.int16}[code]
    codes = gpu.empty((n,), ct, "gpu")
    yf = gpu.empty((n,), np.float32, "gpu")
    args = (xd.data_ptr(), xtype, sx.data_ptr() if sx is not None else None,
            zx.data_ptr() if zx is not None else None, n)
    _qact(gpu, op, *args, codes.data_ptr(), code, so, zo, qmin, qmax)
    _qact(gpu, op, *args, yf.data_ptr(), _C.F32)
    t = yf.numpy()
    _check_float(op, t, O.activation(val, op, PARAM.get(op, 0.0)))
    inv = O.recip_tensor(np.array([s_out], np.float32))[0]
    np.testing.assert_array_equal(codes.numpy(), O.quantize(t, inv, z_out, qmin, qmax, code))


_PAIRS = ["Sigmoid", "Hardswish", "Hardsigmoid", "Tanh", "ELU", "LeakyReLU"]


@pytest.mark.parametrize("name", _PAIRS)
def test_activation_quantizes(gpu, name):
    # lucid/test/unit/quantization/test_module_breadth.py:62-76
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.nn.layers import manual_seed

    Q = gpu.quantization
    manual_seed(0)
    rng = np.random.default_rng(0)
    m = nn.Sequential(nn.Linear(64, 64), getattr(nn, name)()).to("gpu")
    x = gpu.tensor(rng.standard_normal((8, 64)).astype(np.float32), device="gpu")
    yf = m(x).numpy()
    prepared = Q.prepare(m, Q.get_default_qconfig_mapping())
    for _ in range(5):
        prepared(gpu.tensor(rng.standard_normal((8, 64)).astype(np.float32), device="gpu"))
    qm = Q.convert(prepared)
    assert isinstance(qm[1], getattr(nnq, name))
    yq = qm(x).numpy()
    assert np.abs(yf - yq).max() / (np.abs(yf).max() + 1e-9) < 0.1
    sd = qm.state_dict()
    assert "1.scale" in sd and "1.zero_point" in sd


def test_leaky_relu_and_elu_carry_parameters(gpu):
    # test_module_breadth.py:79-89, plus ELU's alpha (activation.py:383-386)
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    rng = np.random.default_rng(1)
    m = nn.Sequential(nn.Linear(8, 8), nn.LeakyReLU(negative_slope=0.2), nn.Linear(8, 8), nn.ELU(alpha=1.5)).to("gpu")
    prepared = Q.prepare(m, Q.get_default_qconfig_mapping())
    for _ in range(3):
        prepared(gpu.tensor(rng.standard_normal((4, 8)).astype(np.float32), device="gpu"))
    qm = Q.convert(prepared)
    assert isinstance(qm[1], nnq.LeakyReLU) and qm[1].negative_slope == pytest.approx(0.2)
    assert isinstance(qm[3], nnq.ELU) and qm[3].alpha == pytest.approx(1.5)


def test_quantized_activation_reads_codes_of_previous_layer(gpu):
    # Linear -> Hardswish inside a quantized region: the activation consumes the Linear's
    # output codes, and its own codes equal the oracle's activation of those values,
    # quantized onto its grid
    import lucid_amd.nn.quantized as nnq

    rng = np.random.default_rng(4)
    x = (rng.standard_normal((16, 40)) * 3).astype(np.float32)
    s_in, z_in = np.float32(0.03), np.float32(128.0)
    q_in = nnq.Quantize(gpu.tensor(s_in, device="gpu"), gpu.tensor(z_in, device="gpu"), gpu.quantization.quint8)
    xq = q_in(gpu.tensor(x, device="gpu"))
    assert xq.is_code_backed
    act = nnq.Hardswish(gpu.tensor(np.float32(0.02), device="gpu"), gpu.tensor(np.float32(20.0), device="gpu"))
    y = act(xq)
    assert y.is_code_backed
    val = O.dequantize(xq.quant_source.codes.numpy(), O.U8S8, s_in, z_in)
    t = O.activation(val, O.ACT_HARDSWISH)
    want = O.quantize(t, O.recip_tensor(np.array([0.02], np.float32))[0], 20.0, 0, 255, O.U8S8)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)
    np.testing.assert_array_equal(y.numpy(), O.dequantize(want, O.U8S8, np.float32(0.02), np.float32(20.0)))


def test_functional_float_ops(gpu):
    import lucid_amd.nn.functional as F

    x = _inputs(1000, 3)
    xd = gpu.tensor(x, device="gpu")
    for fn, op in ((F.sigmoid, O.ACT_SIGMOID), (F.tanh, O.ACT_TANH), (F.hardswish, O.ACT_HARDSWISH),
                   (F.hardsigmoid, O.ACT_HARDSIGMOID)):
        _check_float(op, fn(xd).numpy(), O.activation(x, op))
    _check_float(O.ACT_ELU, F.elu(xd, 1.5).numpy(), O.activation(x, O.ACT_ELU, 1.5))
    _check_float(O.ACT_LEAKY_RELU, F.leaky_relu(xd, 0.2).numpy(), O.activation(x, O.ACT_LEAKY_RELU, 0.2))
