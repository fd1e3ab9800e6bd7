"""``lucid_amd.nn``: the module system and the float layers a quantized model is built from."""

from lucid_amd.nn.module import Module, Parameter
from lucid_amd.nn.layers import (
    ELU,
    AdaptiveAvgPool2d,
    AvgPool2d,
    BatchNorm1d,
    BatchNorm2d,
    BatchNorm3d,
    Conv1d,
    Conv2d,
    Conv3d,
    ConvTranspose1d,
    ConvTranspose2d,
    ConvTranspose3d,
    Embedding,
    EmbeddingBag,
    Flatten,
    Hardsigmoid,
    Hardswish,
    Identity,
    LeakyReLU,
    Linear,
    MaxPool2d,
    ReLU,
    Sequential,
    Sigmoid,
    Tanh,
)

from lucid_amd.nn.rnn import GRU, LSTM, GRUCell, LSTMCell, RNNCell

__all__ = ["Module", "Parameter", "Linear", "Conv2d", "ReLU", "Sequential", "Identity",
           "BatchNorm2d", "Flatten", "Sigmoid", "Tanh", "Hardswish", "Hardsigmoid", "ELU", "LeakyReLU",
           "Embedding", "EmbeddingBag", "MaxPool2d", "AvgPool2d", "AdaptiveAvgPool2d",
           "LSTM", "GRU", "LSTMCell", "GRUCell", "RNNCell", "ConvTranspose2d", "Conv1d", "Conv3d",
           "ConvTranspose1d", "ConvTranspose3d", "BatchNorm1d", "BatchNorm3d"]


def __getattr__(name: str):
    import importlib

    if name in ("quantized", "intrinsic", "functional", "utils"):
        return importlib.import_module(f"lucid_amd.nn.{name}")
    raise AttributeError(f"module 'lucid_amd.nn' has no attribute {name!r}")
