"""``QuantizedLinearMLX`` (lucid/nn/quantized/mlx_linear.py:21-256) on the HIP group-wise GEMM.

Weight-only group-wise quantized Linear: buffers ``packed_weight`` int32
``[out, in*bits/32]``, ``scales`` / ``biases`` ``[out, in/group_size]`` and the float
``bias``; ``forward`` is ``quantized_matmul(x, ...)`` (+ bias, ReLU) in x's dtype.  Like
Lucid's layer it is device-transparent: a host input is moved to the GPU for the call and
the result moved back.  Here bias and ReLU run in the GEMM's epilogue.
"""

from __future__ import annotations

import numpy as np

from lucid_amd._tensor import Tensor, float32, tensor, zeros
from lucid_amd.nn.module import Module
from lucid_amd.quantization._device import on_device
from lucid_amd.quantization._qgemm import quantize, quantized_matmul


class QuantizedLinearMLX(Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True, bits: int = 8,
                 group_size: int = 64, relu: bool = False) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.relu = relu
        packed_cols = in_features * bits // 32
        num_groups = in_features // group_size
        self.register_buffer("packed_weight", zeros((out_features, packed_cols), np.int32))
        self.register_buffer("scales", zeros((out_features, num_groups), float32))
        self.register_buffer("biases", zeros((out_features, num_groups), float32))
        if bias:
            self.register_buffer("bias", tensor(np.zeros(out_features, np.float32)))
        else:
            self.bias = None

    def forward(self, x: Tensor) -> Tensor:
        on_gpu = x.device == "gpu"
        if not on_gpu:
            x = x.to("gpu")
        if any(b is not None and b.device != "gpu" for b in self._buffers.values()):
            self.to("gpu")
        y = quantized_matmul(x, self.packed_weight, self.scales, self.biases, transpose=True,
                             group_size=self.group_size, bits=self.bits, bias=self.bias,
                             relu=self.relu)
        return y if on_gpu else y.to("cpu")

    @classmethod
    def from_float(cls, mod: Module, bits: int = 8, group_size: int = 64,
                   relu: bool = False) -> "QuantizedLinearMLX":
        m = cls(mod.in_features, mod.out_features, bias=mod.bias is not None, bits=bits,
                group_size=group_size, relu=relu)
        packed, scales, biases = quantize(on_device(mod.weight), group_size=group_size, bits=bits)
        m.register_buffer("packed_weight", packed)
        m.register_buffer("scales", scales)
        m.register_buffer("biases", biases)
        if mod.bias is not None:
            m.register_buffer("bias", on_device(mod.bias.detach()))
        return m

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bits={self.bits}, group_size={self.group_size}, relu={self.relu}, backend=hip")
