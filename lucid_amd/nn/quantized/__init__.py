"""``lucid_amd.nn.quantized``: Lucid's quantized inference modules
(lucid/nn/quantized/__init__.py) on the HIP backend.

The int8 layers keep Lucid's buffers and ``state_dict`` layout and run the gfx950 W8A8
MFMA GEMM over integer codes; ``QuantStub`` / ``DeQuantStub`` / ``Quantize`` /
``DeQuantize`` / ``QuantWrapper`` mark the quantized region; ``FloatFunctional`` /
``QFunctional`` carry residual adds and concatenations onto one grid; ``Sigmoid`` /
``Hardswish`` / ``Hardsigmoid`` / ``Tanh`` / ``ELU`` / ``LeakyReLU`` requantize activations;
``Embedding`` / ``EmbeddingBag`` hold per-row int8 tables.
"""

from lucid_amd.nn.quantized.activation import ELU, Hardsigmoid, Hardswish, LeakyReLU, Sigmoid, Tanh
from lucid_amd.nn.quantized.conv import Conv2d
from lucid_amd.nn.quantized.conv_nd import (Conv1d, Conv3d, ConvReLU1d, ConvReLU3d, ConvTranspose1d,
                                            ConvTranspose3d)
from lucid_amd.nn.quantized.conv_transpose import ConvTranspose2d
from lucid_amd.nn.quantized.functional_module import FloatFunctional, QFunctional
from lucid_amd.nn.quantized.intrinsic import ConvReLU2d, LinearReLU
from lucid_amd.nn.quantized.linear import Linear
from lucid_amd.nn.quantized.mlx_linear import QuantizedLinearMLX
from lucid_amd.nn.quantized.modules import (DeQuantize, DeQuantStub, Quantize, QuantStub,
                                            QuantWrapper)
from lucid_amd.nn.quantized.sparse import Embedding, EmbeddingBag

__all__ = ["Linear", "QuantizedLinearMLX", "Conv2d", "ConvReLU2d", "LinearReLU", "QuantStub", "DeQuantStub", "Quantize", "DeQuantize",
           "QuantWrapper", "FloatFunctional", "QFunctional", "Sigmoid", "Hardswish", "Hardsigmoid",
           "Tanh", "ELU", "LeakyReLU", "Embedding", "EmbeddingBag", "ConvTranspose2d", "Conv1d", "Conv3d",
           "ConvReLU1d", "ConvReLU3d", "ConvTranspose1d", "ConvTranspose3d"]


def __getattr__(name: str):
    import importlib

    if name == "dynamic":
        return importlib.import_module("lucid_amd.nn.quantized.dynamic")
    raise AttributeError(f"module 'lucid_amd.nn.quantized' has no attribute {name!r}")
