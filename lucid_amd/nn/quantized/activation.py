"""Quantized activations -- ``Sigmoid`` / ``Hardswish`` / ``Hardsigmoid`` / ``Tanh`` / ``ELU``
/ ``LeakyReLU`` (lucid/nn/quantized/activation.py:20-475).

Each is the float activation followed by a fake-quantize onto the calibrated output grid
``(scale, zero_point, qdtype)``: ``convert`` swaps a calibrated float activation inside a
quantized region for one of these so its output is requantized rather than left at full
precision.  Here the activation and the grid snap are one ``lq_qact`` launch: it reads the
integer codes of a code-backed input (the output of a quantized layer) directly and writes
the output codes, so the result is code-backed too.
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import QuantSource, Tensor, empty
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import _QuantizedGridModule, activation_qparams
from lucid_amd.nn.quantized.functional_module import _grid_codes, _operand
from lucid_amd.quantization._device import on_device
from lucid_amd.quantization._qscheme import QDtype, quint8


class _QuantizedActivation(_QuantizedGridModule):
    """Float activation then fake-quant to the calibrated grid (activation.py:20-41)."""

    _op: int = -1

    def __init__(self, scale: Tensor, zero_point: Tensor, qdtype: QDtype = quint8) -> None:
        super().__init__(scale, zero_point, qdtype)

    def _param(self) -> float:
        """The activation's float parameter (alpha / negative_slope), 0 when it has none."""
        return 0.0

    def _configure(self, mod: Module) -> None:
        """Copy activation-specific parameters from the float module."""

    def forward(self, input: Tensor) -> Tensor:
        """Activate, then fake-quantize to the calibrated grid; code-backed result."""
        name = type(self).__name__
        qmin, qmax = self.qdtype.quant_min, self.qdtype.quant_max
        grid = _grid_codes(qmin, qmax)
        if grid is None:
            raise ValueError(f"{name}: a [{qmin}, {qmax}] grid does not fit 16-bit codes")
        code_type, dt = grid
        ptr, xtype, xs, xz = _operand(input, name)
        s, z = on_device(self.scale), on_device(self.zero_point)
        codes = empty(input.shape, dt, "gpu")
        if input.numel():
            _C.call("lq_qact", self._op, ptr, xtype, xs, xz, input.numel(), self._param(), s.data_ptr(),
                    z.data_ptr(), qmin, qmax, code_type, codes.data_ptr(), None)
        return Tensor._code_backed(QuantSource(codes, code_type, s, z, qmin, qmax), input.shape)

    @classmethod
    def from_float(cls, mod: Module) -> "_QuantizedActivation":
        """From a calibrated float activation (reads its output observer)."""
        scale, zero_point, qdtype = activation_qparams(mod)
        obj = cls(scale, zero_point, qdtype)
        obj._configure(mod)
        return obj


class Sigmoid(_QuantizedActivation):
    """Quantized ``nn.Sigmoid`` (activation.py:44-109): ``sigmoid(x)`` then fake-quant; pair
    it with ``FixedQParamsObserver`` (S = 1/256, Z = 0) for the fixed ``[0, 1]`` grid."""

    _op = _C.ACT_SIGMOID


class Hardswish(_QuantizedActivation):
    """Quantized ``nn.Hardswish`` (activation.py:112-174)."""

    _op = _C.ACT_HARDSWISH


class Hardsigmoid(_QuantizedActivation):
    """Quantized ``nn.Hardsigmoid`` (activation.py:177-241)."""

    _op = _C.ACT_HARDSIGMOID


class Tanh(_QuantizedActivation):
    """Quantized ``nn.Tanh`` (activation.py:244-306); fixed-qparams grid ``[-1, 1]``."""

    _op = _C.ACT_TANH


class ELU(_QuantizedActivation):
    """Quantized ``nn.ELU`` (activation.py:309-390); carries ``alpha`` across convert."""

    _op = _C.ACT_ELU
    alpha: float = 1.0

    def _configure(self, mod: Module) -> None:
        self.alpha = float(getattr(mod, "alpha", 1.0))

    def _param(self) -> float:
        return float(np.float32(self.alpha))


class LeakyReLU(_QuantizedActivation):
    """Quantized ``nn.LeakyReLU`` (activation.py:393-475); carries ``negative_slope``."""

    _op = _C.ACT_LEAKY_RELU
    negative_slope: float = 0.01

    def _configure(self, mod: Module) -> None:
        self.negative_slope = float(getattr(mod, "negative_slope", 0.01))

    def _param(self) -> float:
        return float(np.float32(self.negative_slope))
