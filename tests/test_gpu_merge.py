"""GPU parity of the quantizable merges (FloatFunctional / QFunctional over lq_qmerge)
against the oracle: operands read as floats or straight from integer codes, the float32 op,
then the output grid -- bit-exact codes and materialized floats -- plus the static PTQ flow
of a residual block."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GRIDS = {O.I8: (-128, 127), O.U8S8: (0, 255)}


@pytest.fixture(autouse=True)
def _reference_engine():
    import lucid_amd.backends as backends

    backends.quantized.engine = "reference"
    yield
    backends.quantized.engine = "auto"


def _operand(gpu, x, kind, seed):
    """(device tensor, its float32 value): a float tensor, or a code-backed one."""
    from lucid_amd._tensor import QuantSource, Tensor

    if kind == "f32":
        return gpu.tensor(x, device="gpu"), x
    code = O.I8 if kind == "i8" else O.U8S8
    qmin, qmax = GRIDS[code]
    rng = np.random.default_rng(seed)
    s = np.float32(rng.uniform(0.01, 0.05))
    z = np.float32(0 if code == O.I8 else rng.integers(100, 150))
    codes = O.quantize(x, O.recip_tensor(np.array([s]))[0], z, qmin, qmax, code)
    val = O.dequantize(codes, code, s, z)
    q = QuantSource(gpu.tensor(codes, device="gpu"), code, gpu.tensor(s, device="gpu"),
                    gpu.tensor(z, device="gpu"), qmin, qmax)
    return Tensor._code_backed(q, x.shape), val


def _want_codes(t, s, z, qmin, qmax):
    code = O.I8 if qmin < 0 else O.U8S8
    return O.quantize(t, O.recip_tensor(np.array([s]))[0], z, qmin, qmax, code), code


@pytest.mark.parametrize("op", ["add", "mul", "add_relu", "add_scalar", "mul_scalar"])
@pytest.mark.parametrize("kinds", [("f32", "f32"), ("i8", "u8s8"), ("u8s8", "u8s8"), ("i8", "f32"), ("i8", "i8")])
@pytest.mark.parametrize("qdtype", ["quint8", "qint8"])
@pytest.mark.parametrize("shape", [(3, 5, 37), (2, 48, 7, 16)])
def test_qfunctional_matches_oracle(gpu, op, kinds, qdtype, shape):
    """(2, 48, 7, 16) has a multiple of 16 elements: two operands of one byte code type take
    the 16-bytes-per-thread path; (3, 5, 37) the per-element one."""
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    rng = np.random.default_rng(len(op) * 7 + len(kinds[0]) + len(shape))
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    y = (rng.standard_normal(shape) * 2).astype(np.float32)
    xa, xv = _operand(gpu, x, kinds[0], 1)
    ya, yv = _operand(gpu, y, kinds[1], 2)
    qd = getattr(Q, qdtype)
    s_out, z_out = np.float32(0.037), np.float32(0 if qdtype == "qint8" else 117)
    qf = nnq.QFunctional(gpu.tensor(s_out, device="gpu"), gpu.tensor(z_out, device="gpu"), qd)
    scalar = 0.3
    f32 = np.float32
    if op == "add":
        out, t = qf.add(xa, ya), xv + yv
    elif op == "mul":
        out, t = qf.mul(xa, ya), xv * yv
    elif op == "add_relu":
        out, t = qf.add_relu(xa, ya), xv + yv
        t = np.where(t <= 0, f32(0), t)
    elif op == "add_scalar":
        out, t = qf.add_scalar(xa, scalar), xv + f32(scalar)
    else:
        out, t = qf.mul_scalar(xa, scalar), xv * f32(scalar)
    want, code = _want_codes(t.astype(np.float32), s_out, z_out, qd.quant_min, qd.quant_max)
    assert out.is_code_backed and out.shape == shape
    np.testing.assert_array_equal(out.quant_source.codes.numpy(), want)
    np.testing.assert_array_equal(out.numpy(), O.dequantize(want, code, s_out, z_out))


@pytest.mark.parametrize("dim", [0, 1, 2, -1])
def test_cat_matches_oracle(gpu, dim):
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    rng = np.random.default_rng(dim + 10)
    base = [2, 3, 4]
    shapes = []
    for k in (1, 2, 3):
        s = list(base)
        s[dim] = k
        shapes.append(tuple(s))
    xs = [(rng.standard_normal(s) * 3).astype(np.float32) for s in shapes]
    ops = [_operand(gpu, x, kind, i) for i, (x, kind) in enumerate(zip(xs, ("f32", "i8", "u8s8")))]
    s_out, z_out = np.float32(0.05), np.float32(128)
    qf = nnq.QFunctional(gpu.tensor(s_out, device="gpu"), gpu.tensor(z_out, device="gpu"), Q.quint8)
    out = qf.cat([o[0] for o in ops], dim=dim)
    t = np.concatenate([o[1] for o in ops], axis=dim)
    want, code = _want_codes(t, s_out, z_out, 0, 255)
    np.testing.assert_array_equal(out.quant_source.codes.numpy(), want)
    ff = nnq.FloatFunctional()
    np.testing.assert_array_equal(ff.cat([o[0] for o in ops], dim=dim).numpy(), t)


def test_float_functional_ops(gpu):
    import lucid_amd.nn.quantized as nnq

    rng = np.random.default_rng(3)
    x = rng.standard_normal(1000).astype(np.float32)
    y = rng.standard_normal(1000).astype(np.float32)
    xd, yd = gpu.tensor(x, device="gpu"), gpu.tensor(y, device="gpu")
    ff = nnq.FloatFunctional()
    f32 = np.float32
    np.testing.assert_array_equal(ff.add(xd, yd).numpy(), x + y)
    np.testing.assert_array_equal(ff.mul(xd, yd).numpy(), x * y)
    np.testing.assert_array_equal(ff.add_relu(xd, yd).numpy(), np.where(x + y <= 0, f32(0), x + y))
    np.testing.assert_array_equal(ff.add_scalar(xd, 1.1).numpy(), x + f32(1.1))
    np.testing.assert_array_equal(ff.mul_scalar(xd, -2.5).numpy(), x * f32(-2.5))
    with pytest.raises(ValueError):
        ff.add(xd, gpu.tensor(y[:999], device="gpu"))


def test_residual_block_static_flow(gpu):
    # FloatFunctional observed during calibration, swapped for QFunctional by convert; the
    # skip-add then reads the int8 codes of both branches and requantizes them.
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    rng = np.random.default_rng(9)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.quant = nnq.QuantStub()
            self.fc1 = nn.Linear(48, 48)
            self.relu = nn.ReLU()
            self.fc2 = nn.Linear(48, 48)
            self.skip = nnq.FloatFunctional()
            self.dequant = nnq.DeQuantStub()

        def forward(self, x):
            x = self.quant(x)
            return self.dequant(self.skip.add_relu(self.fc2(self.relu(self.fc1(x))), x))

    model = Block().to("gpu")
    xs = [rng.standard_normal((32, 48)).astype(np.float32) for _ in range(5)]
    float_out = model(gpu.tensor(xs[-1], device="gpu")).numpy()
    prepared = Q.prepare(model, Q.get_minmax_qconfig())
    for x in xs[:4]:
        prepared(gpu.tensor(x, device="gpu"))
    obs = prepared.skip.activation_post_process
    assert np.isfinite(obs.min_val.item()) and obs.max_val.item() > 0
    q = Q.convert(prepared)
    assert isinstance(q.skip, nnq.QFunctional)
    y = q(gpu.tensor(xs[-1], device="gpu")).numpy()
    rel = np.linalg.norm(y - float_out) / np.linalg.norm(float_out)
    assert rel < 0.05, rel
    sd = q.state_dict()
    assert "skip.scale" in sd and "skip.zero_point" in sd
