"""``lucid_amd.nn.quantized.dynamic``: dynamically quantized layers
(lucid/nn/quantized/dynamic/__init__.py), produced by ``quantize_dynamic``."""

from lucid_amd.nn.quantized.dynamic.linear import Linear

__all__ = ["Linear"]
