"""``lucid_amd.nn.quantized.dynamic``: dynamically quantized layers
(lucid/nn/quantized/dynamic/__init__.py), produced by ``quantize_dynamic``."""

from lucid_amd.nn.quantized.dynamic.linear import Linear
from lucid_amd.nn.quantized.dynamic.rnn import GRU, LSTM, GRUCell, LSTMCell, RNNCell

__all__ = ["Linear", "LSTM", "GRU", "LSTMCell", "GRUCell", "RNNCell"]
