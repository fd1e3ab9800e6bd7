"""``PackedSequence`` and its packing helpers (lucid/nn/utils/rnn.py:184-777).

A ``PackedSequence`` is ``(data, batch_sizes, sorted_indices, unsorted_indices)``: ``data``
the time-major concatenation of every sequence's real steps in descending-length order
(``[sum(batch_sizes), *feat]``), ``batch_sizes`` a CPU int64 tensor of the sequences still
alive at each step (non-increasing), the two permutations ``None`` when the batch was already
sorted.  Packing and unpacking are row gathers on the GPU (``lq_embedding`` over float32
rows, indices built on the host from the lengths); padding cells read one extra row that
holds ``padding_value``.
"""

from __future__ import annotations

from typing import NamedTuple, Sequence

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32, tensor
from lucid_amd.quantization._device import require_gpu


class _Fields(NamedTuple):
    data: Tensor
    batch_sizes: Tensor
    sorted_indices: Tensor | None
    unsorted_indices: Tensor | None


def _ints(v) -> list[int]:
    if isinstance(v, Tensor):
        return [int(x) for x in np.asarray(v.numpy()).reshape(-1)]
    return [int(x) for x in v]


def _inverse(perm: list[int]) -> list[int]:
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return inv


class PackedSequence(_Fields):
    """Compact batch of variable-length sequences (lucid/nn/utils/rnn.py:184-260)."""

    def __new__(cls, data: Tensor, batch_sizes, sorted_indices=None, unsorted_indices=None):
        sizes = _ints(batch_sizes)
        if not sizes or sizes[-1] <= 0 or any(a < b for a, b in zip(sizes, sizes[1:])):
            raise ValueError(f"batch_sizes must be a non-empty, non-increasing run of positive counts, got {sizes}")
        if sum(sizes) != int(data.shape[0]):
            raise ValueError(f"batch_sizes sums to {sum(sizes)} but the packed data has {int(data.shape[0])} rows")
        bs = tensor(np.asarray(sizes, np.int64))
        if sorted_indices is not None:
            perm = _ints(sorted_indices)
            if sorted(perm) != list(range(sizes[0])):
                raise ValueError(f"sorted_indices must be a permutation of the batch, got {perm}")
            sorted_indices = tensor(np.asarray(perm, np.int64))
            if unsorted_indices is None:
                unsorted_indices = tensor(np.asarray(_inverse(perm), np.int64))
        return super().__new__(cls, data, bs, sorted_indices, unsorted_indices)

    @property
    def sizes(self) -> list[int]:
        return _ints(self.batch_sizes)


def _gather_rows(table: Tensor, rows: int, D: int, idx: list[int]) -> Tensor:
    """out[i] = table[idx[i]] for a float32 [rows, D] table (GPU)."""
    out = empty((len(idx), D), float32, "gpu")
    if idx and D:
        ix = tensor(np.asarray(idx, np.int32), device="gpu")
        _C.call("lq_embedding", table.data_ptr(), _C.F32, None, None, rows, D, ix.data_ptr(), _C.I32, len(idx),
                out.data_ptr(), None)
    return out


def pack_padded_sequence(input: Tensor, lengths, batch_first: bool = False, enforce_sorted: bool = True):
    """Pack a padded ``(T, B, *)`` (or ``(B, T, *)``) batch (lucid/nn/utils/rnn.py:394-486)."""
    require_gpu(input, "pack_padded_sequence")
    if input.ndim < 2:
        raise ValueError(f"pack_padded_sequence: input needs a time and a batch axis, got shape {tuple(input.shape)}")
    if input.numel() == 0:
        raise ValueError(f"pack_padded_sequence: cannot pack an empty tensor (shape {tuple(input.shape)})")
    if input.dtype != float32:
        raise TypeError("pack_padded_sequence: float32 input expected")
    shape = tuple(int(s) for s in input.shape)
    T, B = (shape[1], shape[0]) if batch_first else (shape[0], shape[1])
    feat = shape[2:]
    F = int(np.prod(feat, dtype=np.int64)) if feat else 1
    lens = _ints(lengths)
    if len(lens) != B:
        raise ValueError(f"pack_padded_sequence: {len(lens)} lengths for a batch of {B}")
    if any(n <= 0 or n > T for n in lens):
        raise ValueError(f"pack_padded_sequence: lengths must lie in [1, {T}], got {lens}")
    order = list(range(B))
    sorted_t = None
    if enforce_sorted:
        if any(a < b for a, b in zip(lens, lens[1:])):
            raise ValueError("`lengths` array must be sorted in decreasing order when `enforce_sorted` is True. "
                             "You can pass `enforce_sorted=False` to pack_padded_sequence and/or pack_sequence "
                             "to sidestep this requirement if you do not need ONNX exportability.")
    else:
        order = sorted(range(B), key=lambda i: -lens[i])
        sorted_t = order
    slens = [lens[i] for i in order]
    sizes = [sum(1 for n in slens if n > t) for t in range(slens[0])]
    idx = []
    for t, bs in enumerate(sizes):
        for j in range(bs):
            b = order[j]
            idx.append(b * T + t if batch_first else t * B + b)
    data = _gather_rows(input.reshape(T * B, F), T * B, F, idx).reshape(len(idx), *feat)
    return PackedSequence(data, sizes, sorted_t)


def pad_packed_sequence(sequence: PackedSequence, batch_first: bool = False, padding_value: float = 0.0,
                        total_length: int | None = None):
    """Unpack to a padded batch in the original order and the lengths (rnn.py:487-593)."""
    data = sequence.data
    require_gpu(data, "pad_packed_sequence")
    sizes = sequence.sizes
    longest = len(sizes)
    if total_length is not None and total_length < longest:
        raise ValueError(f"Expected total_length to be at least the length of the longest sequence in input, but got "
                         f"total_length={total_length} and max sequence length being {longest}")
    T = longest if total_length is None else total_length
    B = sizes[0]
    feat = tuple(int(s) for s in data.shape[1:])
    F = int(np.prod(feat, dtype=np.int64)) if feat else 1
    total = int(data.shape[0])
    table = empty((total + 1, F), float32, "gpu")  # the packed rows and one padding row
    if total:
        _C.call("lq_memcpy_d2d", table.data_ptr(), data.data_ptr(), 4 * total * F, None)
    pad_bits = int(np.asarray(np.float32(padding_value)).view(np.uint32))
    _C.call("lq_fill_u32", table.data_ptr() + 4 * total * F, pad_bits, F, None)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    unsort = _ints(sequence.unsorted_indices) if sequence.unsorted_indices is not None else list(range(B))
    slen = [sum(1 for bs in sizes if bs > j) for j in range(B)]  # sorted position j's length
    idx = []
    for i in (range(B) if batch_first else range(T)):
        for k in (range(T) if batch_first else range(B)):
            b, t = (i, k) if batch_first else (k, i)
            j = unsort[b]  # the sorted position of original sequence b
            idx.append(int(offsets[t]) + j if t < slen[j] else total)
    out = _gather_rows(table, total + 1, F, idx).reshape(*((B, T) if batch_first else (T, B)), *feat)
    lengths = tensor(np.asarray([slen[unsort[b]] for b in range(B)], np.int64))
    return out, lengths


def pad_sequence(sequences: Sequence[Tensor], batch_first: bool = False, padding_value: float = 0.0) -> Tensor:
    """Stack variable-length sequences ``[L_i, *feat]`` into one padded batch (rnn.py:594-700)."""
    if not sequences:
        raise ValueError("received an empty list of sequences")
    feat = tuple(int(s) for s in sequences[0].shape[1:])
    F = int(np.prod(feat, dtype=np.int64)) if feat else 1
    T, B = max(int(s.shape[0]) for s in sequences), len(sequences)
    rows = sum(int(s.shape[0]) for s in sequences)
    table = empty((rows + 1, F), float32, "gpu")
    starts, r = [], 0
    for s in sequences:
        require_gpu(s, "pad_sequence")
        if tuple(int(v) for v in s.shape[1:]) != feat:
            raise ValueError("pad_sequence: only the leading time axis may differ")
        n = int(s.shape[0])
        if n:
            _C.call("lq_memcpy_d2d", table.data_ptr() + 4 * r * F, s.data_ptr(), 4 * n * F, None)
        starts.append(r)
        r += n
    _C.call("lq_fill_u32", table.data_ptr() + 4 * rows * F, int(np.asarray(np.float32(padding_value)).view(np.uint32)),
            F, None)
    idx = []
    for i in (range(B) if batch_first else range(T)):
        for k in (range(T) if batch_first else range(B)):
            b, t = (i, k) if batch_first else (k, i)
            idx.append(starts[b] + t if t < int(sequences[b].shape[0]) else rows)
    return _gather_rows(table, rows + 1, F, idx).reshape(*((B, T) if batch_first else (T, B)), *feat)


def pack_sequence(sequences: Sequence[Tensor], enforce_sorted: bool = True) -> PackedSequence:
    """Pack a list of variable-length sequences (rnn.py:777)."""
    lengths = [int(s.shape[0]) for s in sequences]
    return pack_padded_sequence(pad_sequence(sequences), lengths, enforce_sorted=enforce_sorted)
