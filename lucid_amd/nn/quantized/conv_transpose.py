"""Quantized ``ConvTranspose2d`` (lucid/nn/quantized/conv_transpose.py:45-631).

Buffers as Lucid's: ``weight_int8`` int8 ``[in, out / groups, kh, kw]`` quantized per
channel along axis 1 (``weight_scale`` / ``weight_zero_point`` of length ``out / groups``,
per-channel symmetric), float ``bias`` ``[out]``, the output grid's 0-d ``scale`` /
``zero_point``; ``stride``, ``padding``, ``output_padding``, ``dilation``, ``groups``,
``weight_ch_axis = 1`` and ``out_qdtype`` as attributes.  Lucid's forward is
``fake_quant(conv_transpose2d(x, dequantize(weight_int8), bias))``.

Here the layer is an int8 convolution: the input is spread by the stride with the activation
zero point in the gaps (``lq_stride_expand``), then the implicit-GEMM ``lq_conv2d_i8`` runs at
stride 1 with the flipped, channel-swapped kernel and padding ``d (k - 1) - p`` (+ output
padding), its per-channel scales repeated per group: an exact int32 sum and the W8A8 epilogue
to the output grid's codes.  A float input takes the literal path (dequantized kernel, float
transposed convolution, fake-quantize).  The expansion spends (stride^2 - 1) / stride^2 of the
MACs on zero rows; a per-phase decomposition would avoid them.
"""

from __future__ import annotations

import numpy as np

from lucid_amd._tensor import Tensor, tensor, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import activation_qparams
from lucid_amd.nn.quantized.conv import Conv2d
from lucid_amd.quantization._device import on_device, require_gpu
from lucid_amd.quantization._qscheme import QDtype, per_channel_symmetric, qint8, quint8


def _pair(v) -> tuple[int, int]:
    if isinstance(v, (tuple, list)):
        return (int(v[0]), int(v[1])) if len(v) > 1 else (int(v[0]), int(v[0]))
    return int(v), int(v)


class ConvTranspose2d(Module):
    """Quantized 2-D transposed convolution with a calibrated output grid."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0, output_padding=0,
                 dilation=1, groups: int = 1, bias: bool = True) -> None:
        super().__init__()
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride, self.padding = _pair(kernel_size), _pair(stride), _pair(padding)
        self.output_padding, self.dilation, self.groups = _pair(output_padding), _pair(dilation), groups
        self.out_qdtype: QDtype = quint8
        self.weight_ch_axis = 1
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

    def _equivalent(self, H: int, W: int) -> tuple[Conv2d, tuple[int, int, int, int]]:
        """The stride-1 int8 convolution this layer is over its stride-expanded input (cached
        per buffer set): flipped / channel-swapped codes, scales repeated per group."""
        pads, _, _ = F.convt_geometry(H, W, self.kernel_size, self.stride, self.padding, self.output_padding,
                                      self.dilation)
        key = (id(self.weight_int8), id(self.weight_scale), id(self.weight_zero_point), id(self.bias),
               id(self.scale), id(self.zero_point), self.out_qdtype, pads)
        cache = self.__dict__.get("_eq")
        if cache is None or cache[0] != key:
            codes = F.convt_kernel(self.weight_int8.numpy(), self.groups)
            conv = Conv2d(self.in_channels, self.out_channels, self.kernel_size, 1, 0, self.dilation, self.groups,
                          bias=self.bias is not None)
            conv.padding = pads
            conv.weight_ch_axis = 0
            conv.out_qdtype = self.out_qdtype
            conv.weight_int8 = tensor(codes, device="gpu")
            conv.weight_scale = tensor(np.tile(self.weight_scale.numpy().reshape(-1), self.groups), device="gpu")
            conv.weight_zero_point = tensor(np.tile(self.weight_zero_point.numpy().reshape(-1), self.groups),
                                            device="gpu")
            if self.bias is not None:
                conv.bias = on_device(self.bias)
            conv.scale, conv.zero_point = on_device(self.scale), on_device(self.zero_point)
            self.__dict__["_eq"] = cache = (key, conv)
        return cache[1], pads

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

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, "ConvTranspose2d")
        if x.ndim != 4:
            raise ValueError(f"ConvTranspose2d: NCHW input expected, got {x.shape}")
        conv, _ = self._equivalent(int(x.shape[2]), int(x.shape[3]))
        return conv(F.stride_expand(x, self.stride))

    @classmethod
    def from_float(cls, mod: Module) -> "ConvTranspose2d":
        """Per-channel symmetric int8 weights along axis 1 and the calibrated output grid
        (conv_transpose.py:134-170)."""
        from lucid_amd.quantization._functional import quantize
        from lucid_amd.quantization.observer import PerChannelMinMaxObserver

        if isinstance(mod.padding, str):
            raise NotImplementedError("quantized conv_transpose: string padding is not supported yet")
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

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, stride={self.stride}, "
                f"qdtype={self.out_qdtype.name}")
