"""Quantization schemes and quantized-dtype descriptors.

Same names, members and values as lucid/quantization/_qscheme.py:25-245, since user
code and ``state_dict`` consumers compare against them: four ``QScheme`` members
(granularity x symmetry) and the ``qint8`` / ``quint8`` / ``qint32`` / ``qint4``
grids.  ``quint8`` keeps Lucid's ``int16`` storage dtype so code tensors and
``state_dict`` entries have the dtypes Lucid writes.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass


class QScheme(enum.Enum):
    """Granularity (per tensor / per channel) x symmetry (affine / symmetric)."""

    PER_TENSOR_AFFINE = "per_tensor_affine"
    PER_TENSOR_SYMMETRIC = "per_tensor_symmetric"
    PER_CHANNEL_AFFINE = "per_channel_affine"
    PER_CHANNEL_SYMMETRIC = "per_channel_symmetric"

    @property
    def is_per_channel(self) -> bool:
        return self in (QScheme.PER_CHANNEL_AFFINE, QScheme.PER_CHANNEL_SYMMETRIC)

    @property
    def is_symmetric(self) -> bool:
        return self in (QScheme.PER_TENSOR_SYMMETRIC, QScheme.PER_CHANNEL_SYMMETRIC)


per_tensor_affine = QScheme.PER_TENSOR_AFFINE
per_tensor_symmetric = QScheme.PER_TENSOR_SYMMETRIC
per_channel_affine = QScheme.PER_CHANNEL_AFFINE
per_channel_symmetric = QScheme.PER_CHANNEL_SYMMETRIC


@dataclass(frozen=True)
class QDtype:
    """An integer grid: bit width, signedness, inclusive range and storage dtype name."""

    name: str
    bits: int
    signed: bool
    quant_min: int
    quant_max: int
    storage: str

    def __repr__(self) -> str:
        return f"lucid.quantization.{self.name}"


qint8 = QDtype("qint8", 8, True, -128, 127, "int8")
quint8 = QDtype("quint8", 8, False, 0, 255, "int16")
qint32 = QDtype("qint32", 32, True, -(2**31), 2**31 - 1, "int32")
qint4 = QDtype("qint4", 4, True, -8, 7, "int8")
