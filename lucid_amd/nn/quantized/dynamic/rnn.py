"""Dynamic quantized recurrent layers -- ``LSTM`` / ``GRU`` / ``LSTMCell`` / ``GRUCell`` /
``RNNCell`` (lucid/nn/quantized/dynamic/rnn.py:45-264).

Lucid quantizes every recurrent weight per output row (``PerChannelMinMaxObserver``,
per-channel symmetric ``qint8``), keeps the biases in float, and at forward dequantizes the
weights into a float copy of the module and runs it: the activations stay float32.  Here the
weights stay int8 on the device and every gate product is the weight-only GEMV
(``lq_gemv_w8``: ``x (codes * scale)^T + b`` in float32, the dequantized weight never formed),
inside the same recurrence as the float modules of ``lucid_amd.nn.rnn``.

Buffers follow Lucid's naming (``_buffer_key``, rnn.py:29-33): a parameter ``weight_ih_l0``
becomes ``weight_ih_l0_int8`` + ``weight_ih_l0_scale``, a bias keeps its name.
"""

from __future__ import annotations

import copy

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor
from lucid_amd.nn import rnn as _rnn
from lucid_amd.nn.module import Module
from lucid_amd.quantization._device import on_device, workspace
from lucid_amd.quantization._qscheme import QDtype, per_channel_symmetric, qint8


class _DynamicGates:
    """``x W^T + b`` with the int8 weight and its row scales (weight-only GEMV)."""

    def _gates(self, name: str, x_ptr: int, ldx: int, M: int, K: int, y_ptr: int, ldy: int = 0) -> None:
        codes = self._buffers[f"weight_{name}_int8"]
        if codes.device != "gpu":
            codes = codes.to("gpu")
            self._buffers[f"weight_{name}_int8"] = codes
        scale = on_device(self._buffers[f"weight_{name}_scale"])
        b = self._buffers.get(f"bias_{name}")
        b = on_device(b) if b is not None else None
        N = int(codes.shape[0])
        self._alive = (scale, b)
        wsb = _C.lib().lq_gemv_w8_workspace_size(M, N, K)
        _C.call("lq_gemv_w8", x_ptr, _C.F32, ldx, codes.data_ptr(), K, scale.data_ptr(), None,
                b.data_ptr() if b is not None else None, y_ptr, ldy or N, M, N, K, 0, workspace.get(wsb), wsb, None)


def _quantize_into(qmod: Module, fmod: Module, dtype: QDtype) -> None:
    """Per-row int8 codes + scales of every weight of ``fmod``; biases copied (rnn.py:76-108)."""
    from lucid_amd.quantization._functional import quantize
    from lucid_amd.quantization.observer import PerChannelMinMaxObserver

    for name, param in fmod.named_parameters():
        if param is None:
            continue
        value = on_device(param)
        if name.rpartition(".")[2].startswith("weight"):
            obs = PerChannelMinMaxObserver(ch_axis=0, qscheme=per_channel_symmetric, qdtype=dtype)
            obs(value)
            scale, zero_point = obs.calculate_qparams()
            scale, zero_point = on_device(scale), on_device(zero_point)
            qmod.register_buffer(name + "_int8", quantize(value, scale, zero_point, dtype, ch_axis=0))
            qmod.register_buffer(name + "_scale", scale)
        else:
            qmod.register_buffer(name, value)


class _DynamicRecurrent:
    _FLOAT: type = Module

    @classmethod
    def from_float(cls, mod: Module, dtype: QDtype = qint8):
        """Quantize a float recurrent module's weights (per-channel symmetric int8)."""
        if not isinstance(mod, cls._FLOAT):
            raise TypeError(f"dynamic {cls.__name__}.from_float expects an nn.{cls._FLOAT.__name__}, got "
                            f"{type(mod).__name__}")
        q = cls.__new__(cls)
        Module.__init__(q)
        for k, v in vars(mod).items():   # configuration (sizes, mode, flags), not tensors
            if not k.startswith("_") and not isinstance(v, (Tensor, Module)):
                setattr(q, k, copy.copy(v))
        _quantize_into(q, mod, dtype)
        return q

    def extra_repr(self) -> str:
        return f"{super().extra_repr()}, dynamic=True"


class LSTM(_DynamicRecurrent, _DynamicGates, _rnn._RNNBase):
    _FLOAT = _rnn.LSTM
    forward = _rnn.LSTM.forward


class GRU(_DynamicRecurrent, _DynamicGates, _rnn._RNNBase):
    _FLOAT = _rnn.GRU
    forward = _rnn.GRU.forward


class LSTMCell(_DynamicRecurrent, _DynamicGates, _rnn._CellBase):
    _FLOAT = _rnn.LSTMCell
    forward = _rnn.LSTMCell.forward


class GRUCell(_DynamicRecurrent, _DynamicGates, _rnn._CellBase):
    _FLOAT = _rnn.GRUCell
    forward = _rnn.GRUCell.forward


class RNNCell(_DynamicRecurrent, _DynamicGates, _rnn._CellBase):
    _FLOAT = _rnn.RNNCell
    forward = _rnn.RNNCell.forward
