"""Quantized ``Conv1d`` / ``Conv3d`` / ``ConvReLU1d`` / ``ConvReLU3d`` and
``ConvTranspose1d`` / ``ConvTranspose3d`` (lucid/nn/quantized/conv.py:182,491;
intrinsic.py:141,344; conv_transpose.py:151,473) on the 2-D int8 convolution.

Buffers and ``state_dict`` keys are Lucid's: ``weight_int8`` int8 ``[out, in / groups, *k]``
(``[in, out / groups, *k]`` for the transposed layers) with per-channel ``weight_scale`` /
``weight_zero_point`` (axis 0; axis 1 for the transposed layers), float ``bias``, the output
grid's 0-d ``scale`` / ``zero_point``.  Each layer keeps an equivalent ``nn.quantized.Conv2d``
(rebuilt when a buffer is replaced or a state dict loaded) and runs its input through it:

* 1-D: the input as a height-1 image, the kernel as ``[out, in / groups, 1, k]``;
* 3-D: the input's depth slices each output depth reads, stacked as channels
  (``lq_depth_gather``), the kernel in the same channel order ``[out, kd in / groups, kh, kw]``,
  the output permuted back to NCDHW (``lq_permute_0213``);
* transposed: the flipped, channel-swapped kernel at stride 1 over the stride-expanded input
  (H / W by ``lq_stride_expand``; the depth expansion folded into the gather).

A code-backed input on an 8-bit grid with symmetric weights therefore takes the int8
implicit-GEMM kernel (exact int32 sums over the same products as the 1-D / 3-D convolution,
the W8A8 epilogue to the output grid's codes); any other input the equivalent layer's literal
float path (dequantized kernel, float convolution, fake-quantize).
"""

from __future__ import annotations

import numpy as np

from lucid_amd._tensor import Tensor, tensor, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import activation_qparams, quantize_weight
from lucid_amd.nn.quantized.conv import Conv2d
from lucid_amd.quantization._device import on_device, require_gpu
from lucid_amd.quantization._qscheme import QDtype, per_channel_symmetric, qint8, quint8


class _QuantizedConvNd(Module):
    """Shared buffers, caching and ``from_float`` of the 1-D / 3-D quantized convolutions."""

    _rank = 1
    _relu = False

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, dilation=1,
                 groups: int = 1, bias: bool = True) -> None:
        super().__init__()
        n = self._rank
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride = F._ntuple(kernel_size, n, "kernel_size"), F._ntuple(stride, n, "stride")
        self.padding = padding if isinstance(padding, str) else F._ntuple(padding, n, "padding")
        self.dilation, self.groups = F._ntuple(dilation, n, "dilation"), groups
        self.padding_str: str | None = None
        self.padding_mode = "zeros"
        self.weight_ch_axis = 0
        self.out_qdtype: QDtype = quint8
        self.register_buffer("weight_int8", zeros((out_channels, in_channels // groups, *self.kernel_size), np.int8))
        self.register_buffer("weight_scale", tensor(np.ones(out_channels, np.float32)))
        self.register_buffer("weight_zero_point", tensor(np.zeros(out_channels, np.float32)))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_channels, np.float32)))
        else:
            self.bias = None
        self.register_buffer("scale", tensor(np.float32(1.0)))
        self.register_buffer("zero_point", tensor(np.float32(0.0)))

    def _key(self) -> tuple:
        return tuple(id(b) for b in (self.weight_int8, self.weight_scale, self.weight_zero_point, self.bias,
                                     self.scale, self.zero_point)) + (self.out_qdtype, self.padding_mode)

    def _equivalent(self) -> Conv2d:
        cache = self.__dict__.get("_eq")
        key = self._key()
        if cache is None or cache[0] != key:
            self.__dict__["_eq"] = cache = (key, self._build())
        return cache[1]

    def _conv2d(self, codes: Tensor, stride, pads, dilation) -> Conv2d:
        conv = Conv2d(int(codes.shape[1]) * self.groups, self.out_channels, tuple(codes.shape[2:]), stride, 0,
                      dilation, self.groups, bias=self.bias is not None)
        conv._relu = self._relu
        conv.padding = pads
        conv.padding_mode = self.padding_mode
        conv.out_qdtype = self.out_qdtype
        conv.weight_int8 = codes
        conv.weight_scale = on_device(self.weight_scale)
        conv.weight_zero_point = on_device(self.weight_zero_point)
        if self.bias is not None:
            conv.bias = on_device(self.bias)
        conv.scale, conv.zero_point = on_device(self.scale), on_device(self.zero_point)
        return conv

    def _codes(self) -> Tensor:
        w = self.weight_int8
        return w if w.device == "gpu" else w.to("gpu")

    def _load_from_state_dict(self, *args, **kwargs) -> None:
        super()._load_from_state_dict(*args, **kwargs)
        self.__dict__.pop("_eq", None)

    def __deepcopy__(self, memo: dict):
        import copy

        clone = type(self).__new__(type(self))
        memo[id(self)] = clone
        for k, v in self.__dict__.items():
            if k != "_eq":
                object.__setattr__(clone, k, copy.deepcopy(v, memo))
        return clone

    @classmethod
    def from_float(cls, mod: Module) -> "_QuantizedConvNd":
        """Quantize a calibrated float convolution (its weight observer and activation observer,
        conv.py:137-172); a fused ``[conv, relu]`` block hands over its inner conv."""
        from lucid_amd.nn.quantized.intrinsic import _wire_inner

        mod = _wire_inner(mod)
        has_bias = mod.bias is not None
        q = cls(mod.in_channels, mod.out_channels, mod.kernel_size, mod.stride, mod.padding, mod.dilation,
                mod.groups, bias=has_bias)
        codes, w_scale, w_zp, ch_axis = quantize_weight(mod)
        q.register_buffer("weight_int8", codes)
        q.register_buffer("weight_scale", w_scale)
        q.register_buffer("weight_zero_point", w_zp)
        q.weight_ch_axis = ch_axis
        q.padding_str = getattr(mod, "_padding_str", None)
        q.padding_mode = getattr(mod, "padding_mode", "zeros")
        if has_bias:
            q.register_buffer("bias", on_device(mod.bias.detach()))
        s, z, qd = activation_qparams(mod)
        q.register_buffer("scale", s)
        q.register_buffer("zero_point", z)
        q.out_qdtype = qd
        return q

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, qdtype={self.out_qdtype.name}")


class Conv1d(_QuantizedConvNd):
    """int8-kernel 1-D convolution with a calibrated output grid."""

    _rank = 1

    def _build(self) -> Conv2d:
        (pl, pr), = F.conv_padding_nd(self.padding_str or self.padding, self.kernel_size, self.dilation)
        Cout, Cg, K = (int(v) for v in self.weight_int8.shape)
        return self._conv2d(self._codes().reshape(Cout, Cg, 1, K), (1, self.stride[0]), (0, 0, pl, pr),
                            (1, self.dilation[0]))

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if x.ndim != 3:
            raise ValueError(f"{type(self).__name__}: NCL input expected, got {x.shape}")
        N, C, Lx = (int(v) for v in x.shape)
        y = self._equivalent()(x.reshape(N, C, 1, Lx))
        return y.reshape(N, self.out_channels, int(y.shape[3]))


class Conv3d(_QuantizedConvNd):
    """int8-kernel 3-D convolution with a calibrated output grid."""

    _rank = 3

    def _build(self) -> Conv2d:
        pads = F.conv_padding_nd(self.padding_str or self.padding, self.kernel_size, self.dilation)
        (pt, pb), (pl, pr) = pads[1], pads[2]
        return self._conv2d(F.gathered_kernel(self._codes()), self.stride[1:], (pt, pb, pl, pr), self.dilation[1:])

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if x.ndim != 5:
            raise ValueError(f"{type(self).__name__}: NCDHW input expected, got {x.shape}")
        (pdf, _), _, OD = F.conv3d_geometry(x.shape, self.kernel_size, self.stride, self.padding_str or self.padding,
                                             self.dilation)
        xg = F.depth_gather(x, self.groups, self.kernel_size[0], OD, self.stride[0], pdf, self.dilation[0], 1,
                            self.padding_mode)
        return F.permute_depth(self._equivalent()(xg), int(x.shape[0]), OD)


class ConvReLU1d(Conv1d):
    """Quantized Conv1d with a fused ReLU."""

    _relu = True


class ConvReLU3d(Conv3d):
    """Quantized Conv3d with a fused ReLU."""

    _relu = True


class _QuantizedConvTransposeNd(_QuantizedConvNd):
    """Transposed 1-D / 3-D: weights [in, out / groups, *k] per channel along axis 1."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, output_padding=0,
                 dilation=1, groups: int = 1, bias: bool = True) -> None:
        Module.__init__(self)
        n = self._rank
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride = F._ntuple(kernel_size, n, "kernel_size"), F._ntuple(stride, n, "stride")
        self.padding, self.output_padding = F._ntuple(padding, n, "padding"), F._ntuple(output_padding, n, "output_padding")
        self.dilation, self.groups = F._ntuple(dilation, n, "dilation"), groups
        self.padding_str, self.padding_mode = None, "zeros"
        self.weight_ch_axis = 1
        self.out_qdtype: QDtype = quint8
        n_out = out_channels // groups
        self.register_buffer("weight_int8", zeros((in_channels, n_out, *self.kernel_size), np.int8))
        self.register_buffer("weight_scale", tensor(np.ones(n_out, np.float32)))
        self.register_buffer("weight_zero_point", tensor(np.zeros(n_out, np.float32)))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_channels, np.float32)))
        else:
            self.bias = None
        self.register_buffer("scale", tensor(np.float32(1.0)))
        self.register_buffer("zero_point", tensor(np.float32(0.0)))

    def _conv2d(self, codes: Tensor, stride, pads, dilation) -> Conv2d:
        conv = super()._conv2d(codes, stride, pads, dilation)
        # the equivalent convolution's output channel (g, c) takes channel c's scale
        conv.weight_scale = tensor(np.tile(self.weight_scale.numpy().reshape(-1), self.groups), device="gpu")
        conv.weight_zero_point = tensor(np.tile(self.weight_zero_point.numpy().reshape(-1), self.groups),
                                        device="gpu")
        return conv

    @classmethod
    def from_float(cls, mod: Module) -> "_QuantizedConvTransposeNd":
        """Per-channel symmetric int8 weights along axis 1 and the calibrated output grid
        (conv_transpose.py:134-170)."""
        from lucid_amd.quantization._functional import quantize
        from lucid_amd.quantization.observer import PerChannelMinMaxObserver

        q = cls(mod.in_channels, mod.out_channels, mod.kernel_size, mod.stride, mod.padding, mod.output_padding,
                mod.dilation, mod.groups, bias=mod.bias is not None)
        w = on_device(mod.weight)
        obs = PerChannelMinMaxObserver(ch_axis=1, qscheme=per_channel_symmetric, qdtype=qint8)
        obs(w)
        ws, wz = obs.calculate_qparams()
        ws, wz = on_device(ws), on_device(wz)
        q.register_buffer("weight_int8", quantize(w, ws, wz, qint8, ch_axis=1))
        q.register_buffer("weight_scale", ws)
        q.register_buffer("weight_zero_point", wz)
        if mod.bias is not None:
            q.register_buffer("bias", on_device(mod.bias))
        s, z, qd = activation_qparams(mod)
        q.register_buffer("scale", s)
        q.register_buffer("zero_point", z)
        q.out_qdtype = qd
        return q


class ConvTranspose1d(_QuantizedConvTransposeNd):
    """Quantized 1-D transposed convolution."""

    _rank = 1

    def _build(self) -> Conv2d:
        Cin, Cout_g, K = (int(v) for v in self.weight_int8.shape)
        codes = F.convt_kernel_nd(self.weight_int8.numpy().reshape(Cin, Cout_g, 1, K), self.groups)
        pads, _, _ = F.convt_geometry(1, 1, (1, K), (1, self.stride[0]), (0, self.padding[0]),
                                      (0, self.output_padding[0]), (1, self.dilation[0]))
        return self._conv2d(tensor(codes, device="gpu"), 1, pads, (1, self.dilation[0]))

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if x.ndim != 3:
            raise ValueError(f"{type(self).__name__}: NCL input expected, got {x.shape}")
        N, C, Lx = (int(v) for v in x.shape)
        y = self._equivalent()(F.stride_expand(x.reshape(N, C, 1, Lx), (1, self.stride[0])))
        return y.reshape(N, self.out_channels, int(y.shape[3]))


class ConvTranspose3d(_QuantizedConvTransposeNd):
    """Quantized 3-D transposed convolution."""

    _rank = 3

    def _build(self) -> Conv2d:
        codes = F.convt_kernel_nd(self.weight_int8.numpy(), self.groups)
        pd, pads, _, _, _ = F.convt3d_geometry((1, 1, 1, 1, 1), self.kernel_size, self.stride, self.padding,
                                               self.output_padding, self.dilation)
        return self._conv2d(F.gathered_kernel(tensor(codes, device="gpu")), 1, pads, self.dilation[1:])

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if x.ndim != 5:
            raise ValueError(f"{type(self).__name__}: NCDHW input expected, got {x.shape}")
        pd, _, OD, _, _ = F.convt3d_geometry(x.shape, self.kernel_size, self.stride, self.padding,
                                             self.output_padding, self.dilation)
        return F.convt3d_apply(x, self.stride, pd, self.dilation[0], self.kernel_size[0], OD, self.groups,
                               self._equivalent())
