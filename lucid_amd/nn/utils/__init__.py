"""``lucid_amd.nn.utils``: ``rnn`` (PackedSequence and the packing helpers)."""

from lucid_amd.nn.utils import rnn

__all__ = ["rnn"]
