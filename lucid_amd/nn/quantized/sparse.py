"""Quantized ``Embedding`` / ``EmbeddingBag`` -- per-row int8 tables
(lucid/nn/quantized/sparse.py:28-337).

Buffers as Lucid's: ``weight_int8`` int8 ``[num_embeddings, embedding_dim]``, ``weight_scale``
and ``weight_zero_point`` float32 ``[num_embeddings]`` (per-row, ``ch_axis`` 0).  Lucid's
forward dequantizes the whole table and then looks rows up; here ``lq_embedding`` /
``lq_embedding_bag`` dequantize only the rows they read, in registers, with the same
per-element arithmetic, so the result equals the reference's lookup over the dequantized
table.  ``convert`` swaps float tables without calibration.
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, ones, zeros
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import quantize_weight
from lucid_amd.quantization._device import on_device


def _quantize_table(mod: Module) -> tuple[Tensor, Tensor, Tensor]:
    """Per-row int8 codes of a float table: the qconfig's weight observer, or (no qconfig)
    a per-channel symmetric qint8 observer over rows (sparse.py:146-166, 306-330)."""
    if getattr(mod, "qconfig", None) is None:
        from lucid_amd.quantization._functional import quantize
        from lucid_amd.quantization._qscheme import per_channel_symmetric, qint8
        from lucid_amd.quantization.observer import PerChannelMinMaxObserver

        weight = on_device(mod.weight)
        obs = PerChannelMinMaxObserver(ch_axis=0, qscheme=per_channel_symmetric, qdtype=qint8)
        obs(weight)
        scale, zero_point = obs.calculate_qparams()
        scale, zero_point = on_device(scale), on_device(zero_point)
        codes = quantize(weight, scale, zero_point, qint8, ch_axis=0)
    else:
        codes, scale, zero_point, _ = quantize_weight(mod)
    return codes, scale, zero_point


class _QuantizedTable(Module):
    def __init__(self, num_embeddings: int, embedding_dim: int, padding_idx: int | None) -> None:
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.padding_idx = padding_idx
        self.weight_ch_axis = 0
        self.register_buffer("weight_int8", zeros((num_embeddings, embedding_dim), np.int8))
        self.register_buffer("weight_scale", ones(num_embeddings))
        self.register_buffer("weight_zero_point", zeros(num_embeddings))

    def _table(self) -> tuple[int, int, int, int, int, int]:
        codes = self.weight_int8
        if codes.device != "gpu":
            codes = codes.to("gpu")
            self.weight_int8 = codes
        # Lucid's separate per-row arrays, read as the module holds them (load_state_dict copies
        # into these buffers in place, so a derived copy such as interleaved pairs would go stale)
        s, z = on_device(self.weight_scale), on_device(self.weight_zero_point)
        self._qparams_alive = (s, z)  # keep the device copies alive over the async launch
        return (codes.data_ptr(), _C.I8, s.data_ptr(), z.data_ptr(), int(codes.shape[0]),
                int(codes.shape[1]))

    def _load(self, codes: Tensor, scale: Tensor, zero_point: Tensor) -> None:
        self.register_buffer("weight_int8", codes)
        self.register_buffer("weight_scale", scale)
        self.register_buffer("weight_zero_point", zero_point)


class Embedding(_QuantizedTable):
    """Quantized embedding lookup (sparse.py:28-170): per-row int8, dequantize-on-lookup."""

    def __init__(self, num_embeddings: int, embedding_dim: int, padding_idx: int | None = None) -> None:
        super().__init__(num_embeddings, embedding_dim, padding_idx)

    def forward(self, indices: Tensor) -> Tensor:
        """The dequantized rows of ``indices`` (``[*indices.shape, embedding_dim]``)."""
        return F.table_lookup(*self._table(), indices, "embedding")

    @classmethod
    def from_float(cls, mod: Module) -> "Embedding":
        """Quantize a float ``nn.Embedding``'s table (per-row int8)."""
        qmod = cls(mod.num_embeddings, mod.embedding_dim, padding_idx=mod.padding_idx)
        qmod._load(*_quantize_table(mod))
        return qmod

    def extra_repr(self) -> str:
        return f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}"


class EmbeddingBag(_QuantizedTable):
    """Quantized ``EmbeddingBag`` (sparse.py:173-337): per-row int8 table, pooled lookup
    (``mode`` sum / mean / max; ``per_sample_weights`` with sum)."""

    def __init__(self, num_embeddings: int, embedding_dim: int, mode: str = "mean",
                 padding_idx: int | None = None) -> None:
        super().__init__(num_embeddings, embedding_dim, padding_idx)
        self.mode = mode

    def forward(self, indices: Tensor, offsets: Tensor | None = None, per_sample_weights: Tensor | None = None,
                compressed_indices_mapping: Tensor | None = None) -> Tensor:
        """The pooled dequantized rows of each bag (``[n_bags, embedding_dim]``)."""
        if compressed_indices_mapping is not None:
            raise NotImplementedError("quantized.EmbeddingBag: compressed_indices_mapping is not supported")
        return F.bag_lookup(*self._table(), indices, offsets, self.mode, per_sample_weights, False,
                            self.padding_idx)

    @classmethod
    def from_float(cls, mod: Module) -> "EmbeddingBag":
        """Quantize a float ``nn.EmbeddingBag``'s table (per-row int8)."""
        qmod = cls(mod.num_embeddings, mod.embedding_dim, mode=getattr(mod, "mode", "mean"),
                   padding_idx=getattr(mod, "padding_idx", None))
        qmod._load(*_quantize_table(mod))
        return qmod

    def extra_repr(self) -> str:
        return (f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}, "
                f"mode={self.mode}")
