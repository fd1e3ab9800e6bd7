"""Shared ``from_float`` helpers of the quantized modules (lucid/nn/quantized/_utils.py:29-132).

* :class:`_QuantizedGridModule` -- a module carrying an output grid ``(scale, zero_point,
  qdtype)`` as buffers (``_utils.py:29-45``);
* :func:`quantize_weight` -- weight ``(codes, scale, zero_point, ch_axis)`` from a QAT
  module's ``weight_fake_quant`` or the ``qconfig``'s weight observer (``_utils.py:48-79``);
* :func:`activation_qparams` -- the output grid read from ``activation_post_process``,
  warning when the observer never saw data (``_utils.py:82-105``).

The quantized modules of this backend compute on the GPU, so qparams and codes are
baked on the GPU whatever device the float module was on.
"""

from __future__ import annotations

import warnings

import numpy as np

from lucid_amd._tensor import Tensor
from lucid_amd.nn.module import Module
from lucid_amd.quantization._device import on_device
from lucid_amd.quantization._functional import fake_quantize_to_codes, quantize
from lucid_amd.quantization._qscheme import QDtype, quint8


class _QuantizedGridModule(Module):
    """Base for modules with an output quantization grid ``(scale, zero_point, qdtype)``."""

    def __init__(self, scale: Tensor, zero_point: Tensor, qdtype: QDtype = quint8) -> None:
        super().__init__()
        self.register_buffer("scale", scale)
        self.register_buffer("zero_point", zero_point)
        self.qdtype = qdtype

    def _fake_quant(self, x: Tensor) -> Tensor:
        """``x`` fake-quantized onto the grid; the result is code-backed, so a quantized
        layer that follows reads the integer codes instead of the floats."""
        return fake_quantize_to_codes(x, self.scale, self.zero_point, self.qdtype.quant_min,
                                      self.qdtype.quant_max)


def quantize_weight(mod: Module) -> tuple[Tensor, Tensor, Tensor, int]:
    """``(codes, scale, zero_point, ch_axis)`` of ``mod.weight``.

    A QAT module's ``weight_fake_quant`` is refreshed on the current weight and its qparams
    reused; a PTQ float module runs its ``qconfig.weight()`` observer over the weight now.
    """
    weight = on_device(mod.weight)
    wfq = getattr(mod, "weight_fake_quant", None)
    if wfq is not None:
        wfq(weight)
        scale, zero_point = wfq.calculate_qparams()
        qdtype, ch_axis = wfq.qdtype, wfq.ch_axis
    else:
        qconfig = getattr(mod, "qconfig", None)
        if qconfig is None:
            raise RuntimeError(f"{type(mod).__name__} has no qconfig: run prepare() first or "
                               "set .qconfig")
        wobs = qconfig.weight()
        wobs(weight)
        scale, zero_point = wobs.calculate_qparams()
        qdtype, ch_axis = wobs.qdtype, wobs.ch_axis
    scale, zero_point = on_device(scale), on_device(zero_point)
    codes = quantize(weight, scale, zero_point, qdtype, ch_axis=ch_axis)
    return codes, scale, zero_point, (ch_axis if ch_axis is not None else 0)


def activation_qparams(mod: Module) -> tuple[Tensor, Tensor, QDtype]:
    """The output ``(scale, zero_point, qdtype)`` of ``mod.activation_post_process``."""
    obs = mod.activation_post_process
    min_val = getattr(obs, "min_val", None)
    if isinstance(min_val, Tensor) and bool(np.isinf(min_val.numpy()).any()):
        warnings.warn(
            f"Quantizing {type(mod).__name__} whose activation observer never saw data -- run "
            "calibration through the prepared model before convert(), or the quantized output "
            "collapses to a near-zero grid.",
            stacklevel=3,
        )
    scale, zero_point = obs.calculate_qparams()
    return on_device(scale), on_device(zero_point), obs.qdtype
