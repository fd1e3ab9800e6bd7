"""Quantized fused blocks (lucid/nn/quantized/intrinsic.py:23-341): ``LinearReLU``,
``ConvReLU2d``.

Each is its base layer with ReLU applied before the output grid; on the int8 path the ReLU
runs in the GEMM / conv epilogue (``y <= 0 -> +0`` before requantizing).  ``from_float``
accepts the float fused block (an ``nn.Sequential`` of ``[layer, relu]``), whose ``qconfig``
and observer move onto the inner layer first (``_wire_inner``, intrinsic.py:23-37).
"""

from __future__ import annotations

from lucid_amd.nn.layers import Sequential
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized.conv import Conv2d
from lucid_amd.nn.quantized.linear import Linear


def _wire_inner(mod: Module) -> Module:
    """The weighted child of a float fused block, carrying the block's qparams."""
    if not isinstance(mod, Sequential):
        return mod
    inner = mod[0]
    inner.qconfig = mod.qconfig
    inner.activation_post_process = mod.activation_post_process
    return inner


class LinearReLU(Linear):
    """Quantized Linear with a fused ReLU."""

    _relu = True

    @classmethod
    def from_float(cls, mod: Module) -> "LinearReLU":
        return super().from_float(_wire_inner(mod))


class ConvReLU2d(Conv2d):
    """Quantized Conv2d with a fused ReLU."""

    _relu = True

    @classmethod
    def from_float(cls, mod: Module) -> "ConvReLU2d":
        return super().from_float(_wire_inner(mod))
