"""``QParams`` and ``calculate_qparams`` (lucid/quantization/_qparams.py:22-205).

``calculate_qparams`` runs as one device kernel over the range tensors
(``lq_calc_qparams_f32``), elementwise, so scalar ranges give per-tensor and
length-C ranges give per-channel parameters, exactly as the reference's chain of
0-d tensor ops does:

* range extended to include zero: ``min = minimum(min, 0)``, ``max = maximum(max, 0)``;
* affine: ``s = max((max - min) / (qmax - qmin), eps)``,
  ``z = clip(qmin - round(min / s), qmin, qmax)``;
* symmetric: ``s = max(max(|min|, |max|) / ((qmax - qmin) / 2), eps)``,
  ``z = 0`` (signed) or ``(qmax + qmin + 1) // 2`` (unsigned).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Union

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32
from lucid_amd.quantization._device import on_device, scalar_tensor
from lucid_amd.quantization._qscheme import QDtype, QScheme

_RangeLike = Union[Tensor, float]


@dataclass(frozen=True)
class QParams:
    scale: Tensor
    zero_point: Tensor
    qscheme: QScheme
    qdtype: QDtype
    ch_axis: int | None = None


def calculate_qparams(min_val: _RangeLike, max_val: _RangeLike, qscheme: QScheme, qdtype: QDtype,
                      eps: float = 1e-8) -> tuple[Tensor, Tensor]:
    """``(scale, zero_point)`` float32 device tensors shaped like the ranges."""
    mn = on_device(min_val) if isinstance(min_val, Tensor) else scalar_tensor(min_val)
    mx = on_device(max_val) if isinstance(max_val, Tensor) else scalar_tensor(max_val)
    if mn.shape != mx.shape:
        raise ValueError(f"min/max shapes differ: {mn.shape} vs {mx.shape}")
    scale = empty(mn.shape, float32, "gpu")
    zp = empty(mn.shape, float32, "gpu")
    n = mn.numel()
    if n:
        _C.call("lq_calc_qparams_f32", mn.data_ptr(), mx.data_ptr(), n, int(qscheme.is_symmetric),
                int(qdtype.signed), qdtype.quant_min, qdtype.quant_max, float(np.float32(eps)),
                scale.data_ptr(), zp.data_ptr(), None)
    return scale, zp
