"""Dynamic quantized ``Linear`` (lucid/nn/quantized/dynamic/linear.py:36-113).

Per forward, Lucid measures the input range, derives per-tensor affine ``quint8`` qparams,
fake-quantizes ``x`` onto them, dequantizes the per-channel int8 weight and runs a float
``F.linear`` (linear.py:85-92).  Here the same forward runs on one stream, with no host
round-trip:

1. ``lq_dynamic_quantize_f32``: ``x.min()`` / ``x.max()`` (observer, replace mode), ``(sx, zx)``
   with Lucid's per-tensor affine rule, and the codes of ``x`` (unsigned grids stored as
   ``c - 128``) -- one launch for up to 16384 elements (a decode step), else the three
   launches ``lq_minmax_f32`` -> ``lq_calc_qparams_f32`` -> ``lq_quantize_per_tensor_f32``,
   with the same bits;
2. ``lq_gemm_w8a8`` (``LQ_EPI_A_U8S8``): ``y = fl32(fl32(acc * fl32(sx * sw[n])) + b[n])``
   over the exact int32 ``acc = sum_k (qx - zx) * qw``.

The float32 output equals Lucid's float composition up to the float GEMM's summation
rounding (the int32 accumulator here is exact).
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32, tensor, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized.linear import _WeightedQuantized
from lucid_amd.quantization._device import on_device, require_gpu, workspace
from lucid_amd.quantization._functional import fake_quantize, quantize
from lucid_amd.quantization._gemm import gemm_w8a8, gemv_w8
from lucid_amd.quantization._qparams import calculate_qparams
from lucid_amd.quantization._qscheme import (QDtype, per_channel_symmetric, per_tensor_affine,
                                             qint8, quint8)


_EPS = float(np.float32(1e-8))  # calculate_qparams' default eps, as the float32 kernels read it


def dynamic_qparams(x: Tensor, qdtype: QDtype) -> tuple[Tensor, Tensor]:
    """``calculate_qparams(x.min(), x.max(), per_tensor_affine, qdtype)`` on the device."""
    mn = empty((), float32, "gpu")
    mx = empty((), float32, "gpu")
    n = x.numel()
    ws_bytes = _C.lib().lq_minmax_workspace_size(n)
    _C.call("lq_minmax_f32", x.data_ptr() if n else None, n, mn.data_ptr(), mx.data_ptr(),
            _C.OBS_REPLACE, 0.0, workspace.get(ws_bytes), ws_bytes, None)
    return calculate_qparams(mn, mx, per_tensor_affine, qdtype)


class Linear(_WeightedQuantized):
    """int8-weight linear with per-forward dynamic activation quantization."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight_ch_axis = 0
        self.act_qdtype: QDtype = quint8
        self.register_buffer("weight_int8", zeros((out_features, in_features), np.int8))
        self.register_buffer("weight_scale", tensor(np.ones(out_features, np.float32)))
        self.register_buffer("weight_zero_point", tensor(np.zeros(out_features, np.float32)))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_features, np.float32)))
        else:
            self.bias = None

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, "dynamic Linear")
        if x.dtype != float32:
            raise TypeError(f"dynamic Linear: float32 input expected, got {x.dtype}")
        self._device_buffers()
        qd = self.act_qdtype
        if self.weight_int8.dtype == np.int8 and qd.quant_min >= 0 and qd.quant_max <= 255:
            code_type = _C.U8S8
        elif self.weight_int8.dtype == np.int8 and qd.quant_min >= -128 and qd.quant_max <= 127:
            code_type = _C.I8
        else:  # a grid wider than 8 bits: Lucid's float composition on the device
            x_scale, x_zp = dynamic_qparams(x, qd)
            x_q = fake_quantize(x, x_scale, x_zp, qd.quant_min, qd.quant_max)
            if self.weight_int8.dtype == np.int8:
                return gemv_w8(x_q, self._operands(), self.bias)
            return F.linear(x_q, self._dequantized_weight(), self.bias)
        n = x.numel()
        qp = empty((4,), float32, "gpu")  # min, max, scale, zero point
        codes = empty(x.shape, np.int8, "gpu")
        ws = _C.lib().lq_dynamic_quantize_workspace_size(n)
        _C.call("lq_dynamic_quantize_f32", x.data_ptr() if n else None, n, code_type, qd.quant_min,
                qd.quant_max, _EPS, qp.data_ptr(), codes.data_ptr() if n else None,
                workspace.get(ws) if ws else None, ws, None)
        return gemm_w8a8(codes, code_type, Tensor._element_view(qp, 2), Tensor._element_view(qp, 3),
                         self._operands(), self.bias, _C.OUT_F32)

    @classmethod
    def from_float(cls, mod: Module, dtype: QDtype = qint8) -> "Linear":
        """Quantize a float ``Linear``'s weight per output channel (symmetric, no calibration)."""
        from lucid_amd.quantization.observer import PerChannelMinMaxObserver

        qmod = cls(mod.in_features, mod.out_features, bias=mod.bias is not None)
        weight = on_device(mod.weight)
        obs = PerChannelMinMaxObserver(ch_axis=0, qscheme=per_channel_symmetric, qdtype=dtype)
        obs(weight)
        scale, zero_point = obs.calculate_qparams()
        qmod.register_buffer("weight_int8", quantize(weight, scale, zero_point, dtype, ch_axis=0))
        qmod.register_buffer("weight_scale", scale)
        qmod.register_buffer("weight_zero_point", zero_point)
        if mod.bias is not None:
            qmod.register_buffer("bias", on_device(mod.bias.detach()))
        return qmod

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, dynamic=True"
