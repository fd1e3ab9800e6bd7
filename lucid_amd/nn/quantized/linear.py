"""Quantized ``Linear`` (lucid/nn/quantized/linear.py:37-242) on the int8 MFMA GEMM.

Buffers and ``state_dict`` keys are Lucid's: ``weight_int8`` int8 ``[out, in]``,
``weight_scale`` / ``weight_zero_point`` float32 ``[out]``, float ``bias``, and the output
grid's 0-d ``scale`` / ``zero_point``; ``weight_ch_axis`` and ``out_qdtype`` are plain
attributes.

Lucid's forward is ``fake_quant(act(F.linear(x, dequantize(weight_int8), bias)))``
(linear.py:206-215).  When ``x`` is code-backed -- the output of a ``Quantize`` stub or
of another quantized layer, i.e. already on an 8-bit grid -- the same layer here is one
W8A8 GEMM over the codes:

    acc = sum_k (qx - zx)(qw - zw)                      exact int32
    y   = fl32(fl32(float(acc) * fl32(sx * sw[n])) + b[n]),  ReLU for LinearReLU
    out = clip(round(y * fl32(1 / S)) + Z, qmin, qmax)       codes of the output grid

and the result is a code-backed tensor whose float values are ``(out - Z) * S``.  It
equals Lucid's float composition except where the float GEMM's rounding moves ``y``
across a rounding boundary of the output grid (one code apart; measured in the tests).
A plain float ``x`` (not on a grid) takes Lucid's literal composition on the GPU: the
weight-only int8 GEMM (``lq_gemv_w8``: float activations against the int8 codes and
per-channel scales, bias and ReLU fused), then fake-quantize onto the output grid.
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, float32, tensor, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import activation_qparams, quantize_weight
from lucid_amd.quantization._device import on_device, require_gpu
from lucid_amd.quantization._functional import dequantize, fake_quantize_to_codes
from lucid_amd.quantization._gemm import WeightCache, code_backed_output, gemm_w8a8, gemv_w8
from lucid_amd.quantization._qscheme import QDtype, quint8


def out_kind_for(qdtype: QDtype) -> tuple[int, int] | None:
    """(GEMM output kind, code type) that stores codes of ``qdtype``'s grid, or None."""
    if qdtype.quant_min >= 0 and qdtype.quant_max <= 255:
        return _C.OUT_QU8S8, _C.U8S8
    if qdtype.quant_min >= -128 and qdtype.quant_max <= 127:
        return _C.OUT_Q8, _C.I8
    return None


class _WeightedQuantized(Module):
    """Device operand cache shared by the int8 Linear layers: codes, scales, code sums,
    the packed decode copy and the dequantized float weight, rebuilt when a buffer is
    replaced or a state dict is loaded."""

    def _operands(self) -> WeightCache:
        key = (id(self.weight_int8), id(self.weight_scale), id(self.weight_zero_point))
        cache = self.__dict__.get("_wcache")
        if cache is None or cache[0] != key:
            w = WeightCache(self.weight_int8, self.weight_scale, self.weight_zero_point)
            self.__dict__["_wcache"] = cache = (key, w)
        return cache[1]

    def _dequantized_weight(self) -> Tensor:
        w = self._operands()
        if getattr(w, "dequantized", None) is None:
            w.dequantized = dequantize(w.codes, w.scale, self.weight_zero_point,
                                       ch_axis=self.weight_ch_axis)
        return w.dequantized

    def _device_buffers(self) -> None:
        """Quantized layers compute on the GPU: move CPU buffers there once."""
        if any(b is not None and b.device != "gpu" for b in self._buffers.values()):
            self.to("gpu")

    def _load_from_state_dict(self, *args, **kwargs) -> None:
        super()._load_from_state_dict(*args, **kwargs)
        self.__dict__.pop("_wcache", None)

    def __deepcopy__(self, memo: dict):
        import copy

        clone = type(self).__new__(type(self))
        memo[id(self)] = clone
        for k, v in self.__dict__.items():
            if k != "_wcache":
                object.__setattr__(clone, k, copy.deepcopy(v, memo))
        return clone


class Linear(_WeightedQuantized):
    """int8-weight linear layer with a calibrated output grid."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight_ch_axis = 0
        self.out_qdtype: QDtype = quint8
        self.register_buffer("weight_int8", zeros((out_features, in_features), np.int8))
        self.register_buffer("weight_scale", tensor(np.ones(out_features, np.float32)))
        self.register_buffer("weight_zero_point", tensor(np.zeros(out_features, np.float32)))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_features, np.float32)))
        else:
            self.bias = None
        self.register_buffer("scale", tensor(np.float32(1.0)))
        self.register_buffer("zero_point", tensor(np.float32(0.0)))

    _relu = False

    def _activation(self, y: Tensor) -> Tensor:
        """Post-linear activation hook (identity; ReLU in the fused variant)."""
        return F.relu(y) if self._relu else y

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        self._device_buffers()
        q = x.quant_source
        kind = out_kind_for(self.out_qdtype)
        if (q is not None and q.code_type in (_C.I8, _C.U8S8) and kind is not None
                and self.scale.numel() == 1 and self.zero_point.numel() == 1):
            out_kind, code_type = kind
            codes = gemm_w8a8(q.codes, q.code_type, q.scale,
                              q.zero_point, self._operands(), self.bias, out_kind,
                              self.scale, self.zero_point, self.out_qdtype.quant_min,
                              self.out_qdtype.quant_max, relu=self._relu)
            return code_backed_output(codes, code_type, self.scale, self.zero_point,
                                      self.out_qdtype.quant_min, self.out_qdtype.quant_max)
        if x.dtype != float32:
            raise TypeError(f"{type(self).__name__}: float32 input expected, got {x.dtype}")
        if self.weight_int8.dtype == np.int8:
            y = gemv_w8(x, self._operands(), self.bias, relu=self._relu)
        else:
            y = self._activation(F.linear(x, self._dequantized_weight(), self.bias))
        return fake_quantize_to_codes(y, self.scale, self.zero_point, self.out_qdtype.quant_min,
                                      self.out_qdtype.quant_max)

    @classmethod
    def from_float(cls, mod: Module) -> "Linear":
        """Quantize a calibrated float ``Linear`` (weight observer + activation observer)."""
        has_bias = mod.bias is not None
        qmod = cls(mod.in_features, mod.out_features, bias=has_bias)
        codes, w_scale, w_zp, ch_axis = quantize_weight(mod)
        qmod.register_buffer("weight_int8", codes)
        qmod.register_buffer("weight_scale", w_scale)
        qmod.register_buffer("weight_zero_point", w_zp)
        qmod.weight_ch_axis = ch_axis
        if has_bias:
            qmod.register_buffer("bias", on_device(mod.bias.detach()))
        a_scale, a_zp, a_qdtype = activation_qparams(mod)
        qmod.register_buffer("scale", a_scale)
        qmod.register_buffer("zero_point", a_zp)
        qmod.out_qdtype = a_qdtype
        return qmod

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"qdtype={self.out_qdtype.name}")
