"""Host-side bfloat16 handling of the tensor class (no GPU): the structured bfloat16 dtype,
float32 <-> bfloat16 conversion (round to nearest even, against the oracle's arithmetic
restatement and torch), and ``tensor(..., dtype=bfloat16)`` / ``Tensor.to(dtype=...)`` on
the host."""

from __future__ import annotations

import numpy as np

import lucid_amd as L
import oracle as O


def test_bf16_conversions_match_oracle_and_torch():
    import torch

    rng = np.random.default_rng(1)
    v = (rng.standard_normal(50000) * np.exp(rng.uniform(-110, 87, 50000))).astype(np.float32)
    v = np.concatenate([v, np.array([0.0, -0.0, np.inf, -np.inf, 1 + 2.0 ** -8, 3.4e38], np.float32)])
    b = L.bf16_from_f32(v)
    assert b.dtype == L.bfloat16 and b.dtype != np.uint16 and b.dtype.itemsize == 2
    np.testing.assert_array_equal(L.bf16_to_f32(b).view(np.uint32), O.bf16_round(v).view(np.uint32))
    t = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(b.view(np.uint16), t)
    n = L.bf16_from_f32(np.array([np.nan, -np.nan], np.float32))
    assert np.isnan(L.bf16_to_f32(n)).all()


def test_tensor_bf16_host_round_trip():
    x = np.array([1.0, 1 + 2.0 ** -8, -3.5, 1e-40], np.float32)
    t = L.tensor(x, dtype=L.bfloat16)
    assert t.dtype == L.bfloat16 and t.shape == (4,)
    f = t.to(dtype=np.float32).numpy()
    np.testing.assert_array_equal(f, O.bf16_round(x))
    h = t.to(dtype=np.float16)
    assert h.dtype == np.float16
    np.testing.assert_array_equal(L.tensor(f).to(dtype=L.bfloat16).numpy().view(np.uint16),
                                  t.numpy().view(np.uint16))
