"""Quantized ``Conv2d`` (lucid/nn/quantized/conv.py:61-488) on the int8 implicit-GEMM kernel.

Buffers and ``state_dict`` keys are Lucid's: ``weight_int8`` int8 ``[Cout, Cin/groups, kh,
kw]``, per-output-channel ``weight_scale`` / ``weight_zero_point``, float ``bias`` and the
output grid's 0-d ``scale`` / ``zero_point``; ``stride``, ``padding``, ``padding_str``,
``padding_mode``, ``dilation``, ``groups``, ``weight_ch_axis`` and ``out_qdtype`` are plain
attributes carried over by ``from_float`` (conv.py:137-172).

Lucid's forward is ``fake_quant(act(conv(x, dequantize(weight_int8), bias)))``.  With a
code-backed input on an 8-bit grid and symmetric weights (zero weight zero points), the same
layer is one ``lq_conv2d_i8``: exact int32 accumulation over the codes (padded taps at the
input's zero point, reflect / replicate / circular padding mapped on the codes), then the
W8A8 epilogue -- per-channel scale, bias, ReLU for ConvReLU2d, requantize -- written as the
output grid's codes (NCHW), returned code-backed.  Any other input takes Lucid's literal
composition on the GPU: the dequantized kernel (cached), the float conv kernel, ReLU,
fake-quantize.
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32, tensor, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import activation_qparams, quantize_weight
from lucid_amd.nn.quantized.linear import out_kind_for
from lucid_amd.quantization._device import on_device, require_gpu, workspace
from lucid_amd.quantization._functional import dequantize, fake_quantize_to_codes
from lucid_amd.quantization._gemm import code_backed_output
from lucid_amd.quantization._qscheme import QDtype, quint8


def _pair(v) -> tuple[int, int]:
    if isinstance(v, (tuple, list)):
        return (int(v[0]), int(v[1])) if len(v) > 1 else (int(v[0]), int(v[0]))
    return int(v), int(v)


class _ConvOperands:
    """Device operands of an int8 kernel: packed weights, code sums, scales; the dequantized
    float kernel for the literal path (built on first use)."""

    def __init__(self, mod: "Conv2d") -> None:
        w = mod.weight_int8 if mod.weight_int8.device == "gpu" else mod.weight_int8.to("gpu")
        self.codes = w
        Cout, Cg, KH, KW = w.shape
        self.scale = on_device(mod.weight_scale).reshape(Cout)
        zp = mod.weight_zero_point.numpy().reshape(-1)
        self.symmetric = bool(np.all(zp == 0))
        nbytes = _C.lib().lq_conv2d_weight_pack_size(Cout, Cg, KH, KW)
        self.packed = empty((max(nbytes, 16),), np.int8, "gpu")
        self.sums = empty((Cout,), np.int32, "gpu")
        _C.call("lq_conv2d_pack_weights_i8", w.data_ptr(), Cout, Cg, KH, KW, self.packed.data_ptr(),
                self.sums.data_ptr(), None)
        self.dequantized = None


class Conv2d(Module):
    """int8-kernel 2-D convolution with a calibrated output grid."""

    _relu = False

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, groups: int = 1, bias: bool = True) -> None:
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = padding if isinstance(padding, str) else _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = groups
        self.padding_str: str | None = None
        self.padding_mode = "zeros"
        self.weight_ch_axis = 0
        self.out_qdtype: QDtype = quint8
        kh, kw = self.kernel_size
        self.register_buffer("weight_int8", zeros((out_channels, in_channels // groups, kh, kw), np.int8))
        self.register_buffer("weight_scale", tensor(np.ones(out_channels, np.float32)))
        self.register_buffer("weight_zero_point", tensor(np.zeros(out_channels, np.float32)))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_channels, np.float32)))
        else:
            self.bias = None
        self.register_buffer("scale", tensor(np.float32(1.0)))
        self.register_buffer("zero_point", tensor(np.float32(0.0)))

    # ----------------------------------------------------------- operand cache
    def _operands(self) -> _ConvOperands:
        key = (id(self.weight_int8), id(self.weight_scale), id(self.weight_zero_point))
        cache = self.__dict__.get("_ccache")
        if cache is None or cache[0] != key:
            self.__dict__["_ccache"] = cache = (key, _ConvOperands(self))
        return cache[1]

    def _load_from_state_dict(self, *args, **kwargs) -> None:
        super()._load_from_state_dict(*args, **kwargs)
        self.__dict__.pop("_ccache", None)
        self.__dict__.pop("_fplan", None)

    def __deepcopy__(self, memo: dict):
        import copy

        clone = type(self).__new__(type(self))
        memo[id(self)] = clone
        for k, v in self.__dict__.items():
            if k not in ("_ccache", "_fplan"):
                object.__setattr__(clone, k, copy.deepcopy(v, memo))
        return clone

    def _pads(self) -> tuple[int, int, int, int]:
        return F.conv_padding(self.padding_str or self.padding, self.kernel_size, self.dilation)

    def _activation(self, y: Tensor) -> Tensor:
        return F.relu(y) if self._relu else y

    # ------------------------------------------------------------------ forward
    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if any(b is not None and b.device != "gpu" for b in self._buffers.values()):
            self.to("gpu")
        if x.ndim != 4:
            raise ValueError(f"{type(self).__name__}: NCHW input expected, got {x.shape}")
        ops = self._operands()
        q = x.quant_source
        kind = out_kind_for(self.out_qdtype)
        if (q is not None and q.code_type in (_C.I8, _C.U8S8) and kind is not None and ops.symmetric
                and self.scale.numel() == 1 and self.zero_point.numel() == 1):
            return self._forward_int8(q, x.shape, ops, kind)
        if x.dtype != float32:
            raise TypeError(f"{type(self).__name__}: float32 input expected, got {x.dtype}")
        if ops.dequantized is None:
            ops.dequantized = dequantize(ops.codes, ops.scale, on_device(self.weight_zero_point),
                                         ch_axis=self.weight_ch_axis)
        y = F.conv2d(x, ops.dequantized, self.bias, self.stride, self.padding_str or self.padding,
                     self.dilation, self.groups, self.padding_mode)
        y = self._activation(y)
        return fake_quantize_to_codes(y, self.scale, self.zero_point, self.out_qdtype.quant_min,
                                      self.out_qdtype.quant_max)

    def _forward_int8(self, q, shape, ops: _ConvOperands, kind) -> Tensor:
        out_kind, code_type = kind
        # the call's geometry (output shape, workspace size, size arguments) depends only on
        # the input shape and the layer's attributes: computed once per key
        key = (shape, self.stride, self.padding, self.padding_str, self.dilation, self.groups, self.padding_mode,
               self.out_qdtype.quant_min, self.out_qdtype.quant_max)
        plan = self.__dict__.get("_fplan")
        if plan is None or plan[0] != key or plan[1] is not ops:
            N, C, H, W = shape
            Cout = self.out_channels
            KH, KW = self.kernel_size
            (sh, sw), (dh, dw) = self.stride, self.dilation
            pt, pb, pl, pr = self._pads()
            OH = (H + pt + pb - dh * (KH - 1) - 1) // sh + 1
            OW = (W + pl + pr - dw * (KW - 1) - 1) // sw + 1
            ws_bytes = (_C.lib().lq_conv2d_i8_workspace_size(N, C, H, W, Cout, KH, KW, sh, sw, pt, pb, pl, pr, dh,
                                                             dw, self.groups) if N else 0)
            geom = (N, C, H, W, ops.packed.data_ptr(), ops.sums.data_ptr(), Cout, KH, KW, sh, sw, pt, pb, pl, pr,
                    dh, dw, self.groups, F.PADDING_MODES[self.padding_mode])
            plan = (key, ops, (N, Cout, OH, OW), ws_bytes, geom)
            self.__dict__["_fplan"] = plan
        oshape, ws_bytes, geom = plan[2], plan[3], plan[4]
        codes = empty(oshape, np.int8, "gpu")
        if oshape[0]:
            b = self.bias
            if b is not None:
                b = on_device(b)
            qd = self.out_qdtype
            _C.call("lq_conv2d_i8", q.codes.data_ptr(), q.code_type, *geom, q.scale.data_ptr(),
                    q.zero_point.data_ptr(), ops.scale.data_ptr(), b.data_ptr() if b is not None else None,
                    self.scale.data_ptr(), self.zero_point.data_ptr(), qd.quant_min, qd.quant_max, out_kind,
                    _C.EPI_RELU if self._relu else 0, codes.data_ptr(), workspace.get(ws_bytes), ws_bytes, None)
        return code_backed_output(codes, code_type, self.scale, self.zero_point,
                                  self.out_qdtype.quant_min, self.out_qdtype.quant_max)

    @classmethod
    def from_float(cls, mod: Module) -> "Conv2d":
        """Quantize a calibrated float ``Conv2d`` (weight observer + activation observer)."""
        has_bias = mod.bias is not None
        qmod = cls(mod.in_channels, mod.out_channels, mod.kernel_size, mod.stride, mod.padding,
                   mod.dilation, mod.groups, bias=has_bias)
        codes, w_scale, w_zp, ch_axis = quantize_weight(mod)
        qmod.register_buffer("weight_int8", codes)
        qmod.register_buffer("weight_scale", w_scale)
        qmod.register_buffer("weight_zero_point", w_zp)
        qmod.weight_ch_axis = ch_axis
        qmod.padding_str = getattr(mod, "_padding_str", None)
        qmod.padding_mode = getattr(mod, "padding_mode", "zeros")
        if has_bias:
            qmod.register_buffer("bias", on_device(mod.bias.detach()))
        a_scale, a_zp, a_qdtype = activation_qparams(mod)
        qmod.register_buffer("scale", a_scale)
        qmod.register_buffer("zero_point", a_zp)
        qmod.out_qdtype = a_qdtype
        return qmod

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, qdtype={self.out_qdtype.name}")
