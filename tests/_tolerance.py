"""Float comparison of the device kernels against the oracle's float64 results, in the
reference test suite's scale-aware convention (lucid/test/_helpers/compare.py:54-86,
``assert_close_to_scale``): ``|got - want| <= atol + rtol * |want|`` elementwise with
``atol = rtol * max|want|`` -- the absolute floor is the largest expected magnitude times
rtol, never looser than rtol allows the largest entry.  fp32 outputs use rtol 1e-5 and fp16
outputs rtol 1e-3, with fp16's subnormal step as the floor.
bfloat16 outputs (no north-star tolerance is stated for them) use rtol 2^-7, two of the
type's ulps at the top of a binade."""

from __future__ import annotations

import numpy as np

F32_RTOL = 1e-5
F16_RTOL = 1e-3
BF16_RTOL = 2.0 ** -7


def assert_close_to_scale(got, want, rtol: float, floor: float = 0.0) -> None:
    a = np.asarray(got, np.float64)
    e = np.asarray(want, np.float64)
    assert a.shape == e.shape, f"shape mismatch: {a.shape} vs {e.shape}"
    scale = float(np.max(np.abs(e), initial=0.0, where=np.isfinite(e)))
    atol = max(rtol * scale, floor)
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    assert not bad.any(), (f"{bad.sum()} of {bad.size} outside rtol {rtol} (atol {atol:.3g}); worst "
                           f"{np.max(np.abs(a - e) / (atol + rtol * np.abs(e))):.3g}x the bound")


def assert_close_f32(got, want) -> None:
    assert_close_to_scale(got, want, F32_RTOL)


def assert_close_f16(got, want) -> None:
    assert_close_to_scale(got, want, F16_RTOL, floor=2.0 ** -24)
