"""Float fused blocks (lucid/nn/intrinsic/modules.py:15-353): ``nn.Sequential`` markers that
``fuse_modules`` emits and ``convert`` maps to their quantized counterparts."""

from __future__ import annotations

from lucid_amd.nn.layers import Conv1d, Conv2d, Conv3d, Linear, ReLU, Sequential


class _FusedModule(Sequential):
    """Base tag of the fused float blocks."""


class LinearReLU(_FusedModule):
    def __init__(self, linear: Linear, relu: ReLU) -> None:
        super().__init__(linear, relu)


class ConvReLU2d(_FusedModule):
    def __init__(self, conv: Conv2d, relu: ReLU) -> None:
        super().__init__(conv, relu)


class ConvReLU1d(_FusedModule):
    def __init__(self, conv: Conv1d, relu: ReLU) -> None:
        super().__init__(conv, relu)


class ConvReLU3d(_FusedModule):
    def __init__(self, conv: Conv3d, relu: ReLU) -> None:
        super().__init__(conv, relu)


__all__ = ["LinearReLU", "ConvReLU1d", "ConvReLU2d", "ConvReLU3d"]
