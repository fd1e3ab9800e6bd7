"""Quantization boundary markers (lucid/nn/quantized/modules.py:28-411).

``QuantStub`` / ``DeQuantStub`` sit in a float model (identity until ``prepare`` hangs an
observer on the stub; a QAT ``FakeQuantize`` observer is applied, modules.py:111-122);
``convert`` turns them into ``Quantize`` (fake-quantize onto the calibrated grid -- here a
code-backed result, so the next quantized layer reads integer codes) and ``DeQuantize``
(identity: activations stay float tensors, modules.py:281-335).  ``QuantWrapper`` wraps a
model as ``quant -> module -> dequant``.
"""

from __future__ import annotations

import numpy as np

from lucid_amd._tensor import Tensor, tensor
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import _QuantizedGridModule
from lucid_amd.quantization._qscheme import QDtype, quint8


class QuantStub(Module):
    """Entry marker of the quantized region (identity in PTQ)."""

    def __init__(self, qconfig: object = None) -> None:
        super().__init__()
        if qconfig is not None:
            self.qconfig = qconfig

    def forward(self, x: Tensor) -> Tensor:
        app = getattr(self, "activation_post_process", None)
        if app is not None and getattr(app, "is_fake_quantize", False) and x.dtype == np.float32:
            return app(x)
        return x


class DeQuantStub(Module):
    """Exit marker of the quantized region (identity)."""

    def __init__(self, qconfig: object = None) -> None:
        super().__init__()
        if qconfig is not None:
            self.qconfig = qconfig

    def forward(self, x: Tensor) -> Tensor:
        return x


class Quantize(_QuantizedGridModule):
    """Fake-quantize float input onto ``(scale, zero_point, qdtype)``; integer tensors pass."""

    def __init__(self, scale: Tensor | float = 1.0, zero_point: Tensor | float = 0.0,
                 qdtype: QDtype = quint8) -> None:
        if not isinstance(scale, Tensor):
            scale = tensor(np.float32(scale))
        if not isinstance(zero_point, Tensor):
            zero_point = tensor(np.float32(zero_point))
        super().__init__(scale, zero_point, qdtype)

    def forward(self, X: Tensor) -> Tensor:
        if X.dtype != np.float32:
            return X
        if self.scale.device != "gpu" or self.zero_point.device != "gpu":
            self.to("gpu")
        return self._fake_quant(X)

    @classmethod
    def from_float(cls, stub: Module) -> "Quantize":
        obs = stub.activation_post_process
        scale, zero_point = obs.calculate_qparams()
        return cls(scale, zero_point, obs.qdtype)

    def extra_repr(self) -> str:
        return f"qdtype={self.qdtype.name}"


class DeQuantize(Module):
    """Exit of the quantized region after ``convert`` (identity)."""

    def forward(self, Xq: Tensor) -> Tensor:
        return Xq

    @classmethod
    def from_float(cls, stub: Module) -> "DeQuantize":
        del stub
        return cls()


class QuantWrapper(Module):
    """``quant -> module -> dequant`` around a float model."""

    def __init__(self, module: Module) -> None:
        super().__init__()
        self.quant = QuantStub()
        self.module = module
        self.dequant = DeQuantStub()

    def forward(self, x: Tensor) -> Tensor:
        return self.dequant(self.module(self.quant(x)))
