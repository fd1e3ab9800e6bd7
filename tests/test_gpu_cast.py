"""GPU parity of ``lq_cast`` (float32 / float16 / bfloat16 conversions, Lucid's astype between
float dtypes, lucid/_C/ops/ufunc/Astype.cpp:42) through the C ABI and ``Tensor.to(dtype=...)``:
bit-exact against numpy's IEEE half conversion and the oracle's bfloat16 rounding, over
normal, subnormal, tie, overflow, infinite and NaN values."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _values() -> np.ndarray:
    rng = np.random.default_rng(9)
    v = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-110, 87, 1 << 16))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 1 + 2.0 ** -11,
                        65504.0, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -134, 3.4e38,
                        1e-45], np.float32)
    with np.errstate(over="ignore"):
        return np.concatenate([special, v, v.astype(np.float16).astype(np.float32)])


def _host(v32: np.ndarray, dst: str) -> np.ndarray:
    """Expected bits of float32 values converted to dst."""
    with np.errstate(over="ignore"):
        if dst == "f16":
            return v32.astype(np.float16).view(np.uint16)
    if dst == "bf16":
        out = O.bf16_round(v32).view(np.uint32) >> 16
        nan = np.isnan(v32)
        out[nan] = (v32.view(np.uint32)[nan] >> 16) | 0x40  # quiet NaN, sign kept
        return out.astype(np.uint16)
    return v32.view(np.uint32)


@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("dst", ["f32", "f16", "bf16"])
def test_cast_pairs_bit_exact(gpu, src, dst):
    from lucid_amd import _C

    code = {"f32": _C.F32, "f16": _C.F16, "bf16": _C.BF16}
    v = _values()
    if src == "f32":
        xs = v
    elif src == "f16":
        with np.errstate(over="ignore"):
            xs = v.astype(np.float16)
    else:
        xs = gpu.bf16_from_f32(v)
    x32 = xs.astype(np.float32) if src != "bf16" else gpu.bf16_to_f32(xs)  # exact widening
    want = _host(x32, dst)
    xd = gpu.tensor(xs, device="gpu")
    y = gpu.empty(v.shape, {"f32": np.float32, "f16": np.float16, "bf16": gpu.bfloat16}[dst], "gpu")
    _C.call("lq_cast", xd.data_ptr(), code[src], y.data_ptr(), code[dst], v.size, None)
    got = y.numpy().view(np.uint32 if dst == "f32" else np.uint16)
    nan = np.isnan(x32)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    # NaN stays NaN (payload bits aside)
    back = got[nan].view(np.float32) if dst == "f32" else (
        got[nan].view(np.float16).astype(np.float32) if dst == "f16" else gpu.bf16_to_f32(got[nan].view(gpu.bfloat16)))
    assert np.isnan(back).all()
    # Tensor.to on the device gives the same bits
    z = xd.to(dtype={"f32": np.float32, "f16": np.float16, "bf16": gpu.bfloat16}[dst])
    np.testing.assert_array_equal(z.numpy().view(got.dtype)[~nan], got[~nan])


def test_cast_rejects(gpu):
    from lucid_amd import _C

    x = gpu.empty((4,), np.float32, "gpu")
    assert _C.lib().lq_cast(x.data_ptr(), _C.I8, x.data_ptr(), _C.F32, 4, None) == -1
    assert _C.lib().lq_cast(x.data_ptr(), _C.F32, x.data_ptr(), _C.F32, -1, None) == -1
    with pytest.raises(gpu.LucidError):
        gpu.tensor(np.zeros(3, np.int8), device="gpu").to(dtype=np.float32)
