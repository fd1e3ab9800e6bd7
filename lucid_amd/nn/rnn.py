"""Recurrent layers -- ``RNNCell`` / ``LSTMCell`` / ``GRUCell`` and the multi-layer,
optionally bidirectional ``LSTM`` / ``GRU`` (lucid/nn/modules/rnn.py), on the GPU.

Each layer and direction computes its input gates for every time step at once
(``x W_ih^T + b_ih``, one matrix product over T x B rows), then walks the time steps: one
product ``h W_hh^T + b_hh`` and one ``lq_rnn_cell`` launch per step, the new hidden state
written straight into the layer's output sequence.  ``batch_first`` is handled by strides
(no transposes).  Parameter names and shapes are Lucid's (``weight_ih_l{k}[_reverse]``
``[G * hidden, in]``, ``weight_hh_l{k}``, ``bias_ih_l{k}``, ``bias_hh_l{k}``; a cell's
``weight_ih`` ...), so ``quantize_dynamic`` finds them.  The matrix products are the float
``lq_linear_f32`` here and the weight-only int8 GEMV in ``nn.quantized.dynamic``.

A ``PackedSequence`` input (``lucid_amd.nn.utils.rnn``) runs the same recurrence over the
packed rows: step t advances the first ``batch_sizes[t]`` sequences (descending lengths, so
the live ones are a prefix), the reverse direction walks the steps backwards so a sequence
joins at its own last step with its initial state, ``h_n`` holds each sequence's state after
its own last step, and an unsorted batch's states are permuted on the way in and out
(lucid/nn/quantized/dynamic/rnn.py:167-197 runs packed input through the float shell).

An LSTM with ``proj_size`` P > 0 (lucid/nn/modules/recurrent_base.py:138-192, the engine's
lucid/_C/backend/cpu/Lstm.h:90-164) carries and emits h = (o tanh(c)) W_hr^T: the cell writes
o tanh(c) [B, H] to a private buffer and one more product ``weight_hr_l{k}`` (no bias) makes
the P-wide state, so ``weight_hh`` is [4H, P], a deeper layer reads D P features and h_0 / h_n
are P wide while c stays H wide.

Not covered: inter-layer dropout (these are inference modules: dropout is the identity in
eval).
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32, tensor
from lucid_amd.nn.module import Module, Parameter
from lucid_amd.quantization._device import require_gpu

_GATES = {"RNN_TANH": 1, "RNN_RELU": 1, "LSTM": 4, "GRU": 3}
_KIND = {"RNN_TANH": _C.RNN_TANH, "RNN_RELU": _C.RNN_RELU, "LSTM": _C.RNN_LSTM, "GRU": _C.RNN_GRU}


def _init_uniform(shape, hidden: int) -> Tensor:
    from lucid_amd.nn import layers

    k = 1.0 / math.sqrt(hidden) if hidden > 0 else 0.0
    return tensor(layers._init_rng.uniform(-k, k, size=shape).astype(np.float32))


class _Recurrent(Module):
    """Shared recurrence; subclasses provide ``_gates(name, x_ptr, ldx, M, K, y_ptr, ldy)``,
    the product ``x W_{name}^T + b_{name}`` for ``name`` = ``ih{suffix}`` / ``hh{suffix}`` /
    ``hr{suffix}`` (the projection, no bias) into rows ``ldy`` apart (0: packed)."""

    mode: str = "LSTM"
    proj_size: int = 0

    def _gates(self, name: str, x_ptr: int, ldx: int, M: int, K: int, y_ptr: int, ldy: int = 0) -> None:
        raise NotImplementedError

    def _rec(self) -> int:
        """The width of the carried (and emitted) hidden state."""
        return self.proj_size if self.proj_size > 0 else self.hidden_size

    def _cell(self, gx_ptr: int, ld_gx: int, gh: Tensor, h: Tensor, c: Tensor | None, B: int, sfx: str,
              y_ptr: int | None, ld_y: int, raw: Tensor | None) -> None:
        """One step of B rows: the cell into h (and y), or, projected, the cell's o tanh(c)
        into ``raw`` and then h = raw W_hr^T into h and y."""
        H, G = self.hidden_size, _GATES[self.mode]
        cp = c.data_ptr() if c is not None else None
        if raw is None:
            _C.call("lq_rnn_cell", _KIND[self.mode], gx_ptr, ld_gx, gh.data_ptr(), G * H, h.data_ptr(), cp, B, H,
                    h.data_ptr(), cp, y_ptr, ld_y, None)
            return
        _C.call("lq_rnn_cell", _KIND[self.mode], gx_ptr, ld_gx, gh.data_ptr(), G * H, raw.data_ptr(), cp, B, H,
                raw.data_ptr(), cp, None, 0, None)
        self._gates("hr" + sfx, raw.data_ptr(), H, B, H, h.data_ptr())
        if y_ptr is not None:   # the same product again, into the output rows
            self._gates("hr" + sfx, raw.data_ptr(), H, B, H, y_ptr, ld_y)

    # -- one recurrent layer over a whole sequence -------------------------------------
    def _layer(self, x: Tensor, T: int, B: int, batch_first: bool, sfx: str, d: int, D: int,
               h: Tensor, c: Tensor | None, out: Tensor) -> None:
        H, G, R = self.hidden_size, _GATES[self.mode], self._rec()
        K = int(x.shape[-1])
        gx = empty((T * B, G * H), float32, "gpu")
        self._gates("ih" + sfx, x.data_ptr(), K, T * B, K, gx.data_ptr())
        gh = empty((B, G * H), float32, "gpu")
        raw = empty((B, H), float32, "gpu") if self.proj_size > 0 else None
        steps = range(T - 1, -1, -1) if d else range(T)
        for t in steps:
            self._gates("hh" + sfx, h.data_ptr(), R, B, R, gh.data_ptr())
            if batch_first:   # rows (b, t) of [B, T, .]
                gx_ptr, ld_gx = gx.data_ptr() + 4 * t * G * H, T * G * H
                y_ptr, ld_y = out.data_ptr() + 4 * (t * D * R + d * R), T * D * R
            else:             # rows (t, b) of [T, B, .]
                gx_ptr, ld_gx = gx.data_ptr() + 4 * t * B * G * H, G * H
                y_ptr, ld_y = out.data_ptr() + 4 * (t * B * D * R + d * R), D * R
            self._cell(gx_ptr, ld_gx, gh, h, c, B, sfx, y_ptr, ld_y, raw)

    def _layer_packed(self, x: Tensor, sizes: list[int], offsets: list[int], sfx: str, d: int, D: int,
                      h: Tensor, c: Tensor | None, out: Tensor) -> None:
        """One layer and direction over packed rows ``x`` [total, K]; writes its column block
        of ``out`` [total, D R]."""
        H, G, R = self.hidden_size, _GATES[self.mode], self._rec()
        K, total = int(x.shape[-1]), int(x.shape[0])
        gx = empty((total, G * H), float32, "gpu")
        self._gates("ih" + sfx, x.data_ptr(), K, total, K, gx.data_ptr())
        gh = empty((sizes[0], G * H), float32, "gpu")
        raw = empty((sizes[0], H), float32, "gpu") if self.proj_size > 0 else None
        steps = range(len(sizes) - 1, -1, -1) if d else range(len(sizes))
        for t in steps:
            bs = sizes[t]
            self._gates("hh" + sfx, h.data_ptr(), R, bs, R, gh.data_ptr())
            self._cell(gx.data_ptr() + 4 * offsets[t] * G * H, G * H, gh, h, c, bs, sfx,
                       out.data_ptr() + 4 * (offsets[t] * D * R + d * R), D * R, raw)

    def _state(self, hx: Tensor | None, idx: int, B: int, W: int | None = None) -> Tensor:
        """A private contiguous [B, W] copy (W = hidden_size by default) of layer-direction
        ``idx`` of ``hx`` (zeros if None)."""
        W = self.hidden_size if W is None else W
        s = empty((B, W), float32, "gpu")
        if hx is None:
            _C.call("lq_fill_u32", s.data_ptr(), 0, B * W, None)
        else:
            _C.call("lq_memcpy_d2d", s.data_ptr(), hx.data_ptr() + 4 * idx * B * W, 4 * B * W, None)
        return s


class _RNNBase(_Recurrent):
    def __init__(self, mode: str, input_size: int, hidden_size: int, num_layers: int = 1, bias: bool = True,
                 batch_first: bool = False, dropout: float = 0.0, bidirectional: bool = False,
                 proj_size: int = 0) -> None:
        super().__init__()
        # the reference's refusals (lucid/nn/modules/recurrent_base.py:138-145)
        if proj_size < 0:
            raise ValueError(f"proj_size must be >= 0, got {proj_size}")
        if proj_size > 0 and mode != "LSTM":
            raise ValueError("proj_size argument is only supported for LSTM, not RNN or GRU")
        if proj_size > 0 and proj_size >= hidden_size:
            raise ValueError(f"proj_size ({proj_size}) must be smaller than hidden_size ({hidden_size})")
        self.mode = mode
        self.input_size, self.hidden_size, self.num_layers = input_size, hidden_size, num_layers
        self.bias, self.batch_first, self.dropout, self.bidirectional = bias, batch_first, dropout, bidirectional
        self.proj_size = proj_size
        G, D, R = _GATES[mode], 2 if bidirectional else 1, self._rec()
        # per layer and direction: weight_ih, weight_hh, bias_ih, bias_hh, weight_hr -- the
        # reference's names, shapes and order (recurrent_base.py:164-194)
        for layer in range(num_layers):
            for d in range(D):
                sfx = f"_l{layer}" + ("_reverse" if d else "")
                in_size = input_size if layer == 0 else D * R
                setattr(self, f"weight_ih{sfx}", Parameter(_init_uniform((G * hidden_size, in_size), hidden_size)))
                setattr(self, f"weight_hh{sfx}", Parameter(_init_uniform((G * hidden_size, R), hidden_size)))
                if bias:
                    setattr(self, f"bias_ih{sfx}", Parameter(_init_uniform((G * hidden_size,), hidden_size)))
                    setattr(self, f"bias_hh{sfx}", Parameter(_init_uniform((G * hidden_size,), hidden_size)))
                if proj_size > 0:
                    setattr(self, f"weight_hr{sfx}", Parameter(_init_uniform((proj_size, hidden_size), hidden_size)))

    def _run_packed(self, packed, hx: Tensor | None, cx: Tensor | None):
        from lucid_amd.nn.utils.rnn import PackedSequence, _gather_rows

        data = packed.data
        require_gpu(data, type(self).__name__)
        if data.dtype != float32 or data.ndim != 2:
            raise TypeError(f"{type(self).__name__}: packed data must be float32 [total, input_size]")
        if int(data.shape[1]) != self.input_size:
            raise ValueError(f"{type(self).__name__}: input size {int(data.shape[1])} != {self.input_size}")
        sizes = packed.sizes
        offsets = [0]
        for bs in sizes[:-1]:
            offsets.append(offsets[-1] + bs)
        B, D, H, L, R = sizes[0], (2 if self.bidirectional else 1), self.hidden_size, self.num_layers, self._rec()
        order = [int(v) for v in packed.sorted_indices.numpy()] if packed.sorted_indices is not None else None

        def permute(st: Tensor | None, perm: list[int] | None, W: int) -> Tensor | None:
            """States [L D, B, W] with their batch axis reordered (row gather)."""
            if st is None or perm is None:
                return st
            if int(np.prod(st.shape)) != L * D * B * W:
                raise ValueError(f"{type(self).__name__}: states must hold {L * D} x {B} x {W} values")
            idx = [ld * B + p for ld in range(L * D) for p in perm]
            return _gather_rows(st, L * D * B, W, idx).reshape(L * D, B, W)

        hx, cx = permute(hx, order, R), permute(cx, order, H)
        self._check_states(hx, cx, L * D, B)
        h_n = empty((L * D, B, R), float32, "gpu")
        c_n = empty((L * D, B, H), float32, "gpu") if self.mode == "LSTM" else None
        layer_in = data
        total = int(data.shape[0])
        for layer in range(L):
            out = empty((total, D * R), float32, "gpu")
            for d in range(D):
                idx = layer * D + d
                h = self._state(hx, idx, B, R)
                c = self._state(cx, idx, B) if self.mode == "LSTM" else None
                self._layer_packed(layer_in, sizes, offsets, f"_l{layer}" + ("_reverse" if d else ""), d, D, h, c,
                                   out)
                self._keep_states(h_n, c_n, idx, B, h, c)
            layer_in = out
        unsort = [int(v) for v in packed.unsorted_indices.numpy()] if packed.unsorted_indices is not None else None
        out_seq = PackedSequence(layer_in, sizes, packed.sorted_indices, packed.unsorted_indices)
        return out_seq, permute(h_n, unsort, R), permute(c_n, unsort, H)

    def _check_states(self, hx: Tensor | None, cx: Tensor | None, LD: int, B: int) -> None:
        """h_0 must hold LD x B x R values (R = proj_size when projected), c_0 LD x B x H."""
        for name, st, W in (("hx", hx, self._rec()), ("cx", cx, self.hidden_size)):
            if st is not None and int(np.prod(st.shape)) != LD * B * W:
                raise ValueError(f"{type(self).__name__}: {name} must hold {LD} x {B} x {W} values, got "
                                 f"shape {tuple(st.shape)}")

    def _keep_states(self, h_n: Tensor, c_n: Tensor | None, idx: int, B: int, h: Tensor, c: Tensor | None) -> None:
        R, H = self._rec(), self.hidden_size
        _C.call("lq_memcpy_d2d", h_n.data_ptr() + 4 * idx * B * R, h.data_ptr(), 4 * B * R, None)
        if c is not None:
            _C.call("lq_memcpy_d2d", c_n.data_ptr() + 4 * idx * B * H, c.data_ptr(), 4 * B * H, None)

    def _run(self, input: Tensor, hx: Tensor | None, cx: Tensor | None):
        from lucid_amd.nn.utils.rnn import PackedSequence

        if isinstance(input, PackedSequence):
            return self._run_packed(input, hx, cx)
        require_gpu(input, type(self).__name__)
        if input.dtype != float32:
            raise TypeError(f"{type(self).__name__}: float32 input expected, got {input.dtype}")
        if input.ndim not in (2, 3):
            raise ValueError(f"{type(self).__name__}: expected a 2-D or 3-D input, got {input.ndim}-D")
        unbatched = input.ndim == 2   # (T, input_size) whatever batch_first says
        x = input.reshape(int(input.shape[0]), 1, int(input.shape[1])) if unbatched else input
        bf = self.batch_first and not unbatched
        T, B = (int(x.shape[1]), int(x.shape[0])) if bf else (int(x.shape[0]), int(x.shape[1]))
        D, H, L, R = (2 if self.bidirectional else 1), self.hidden_size, self.num_layers, self._rec()
        if int(x.shape[-1]) != self.input_size:
            raise ValueError(f"{type(self).__name__}: input size {int(x.shape[-1])} != {self.input_size}")
        self._check_states(hx, cx, L * D, B)
        h_n = empty((L * D, B, R), float32, "gpu")
        c_n = empty((L * D, B, H), float32, "gpu") if self.mode == "LSTM" else None
        layer_in = x
        for layer in range(L):
            out = empty(((B, T, D * R) if bf else (T, B, D * R)), float32, "gpu")
            for d in range(D):
                idx = layer * D + d
                h = self._state(hx, idx, B, R)
                c = self._state(cx, idx, B) if self.mode == "LSTM" else None
                self._layer(layer_in, T, B, bf, f"_l{layer}" + ("_reverse" if d else ""), d, D, h, c, out)
                self._keep_states(h_n, c_n, idx, B, h, c)
            layer_in = out
        out = layer_in
        if unbatched:
            out = out.reshape(T, D * R)
            h_n = h_n.reshape(L * D, R)
            c_n = c_n.reshape(L * D, H) if c_n is not None else None
        return out, h_n, c_n

    def extra_repr(self) -> str:
        s = f"{self.input_size}, {self.hidden_size}"
        if self.num_layers != 1:
            s += f", num_layers={self.num_layers}"
        if self.batch_first:
            s += ", batch_first=True"
        if self.bidirectional:
            s += ", bidirectional=True"
        if self.proj_size > 0:
            s += f", proj_size={self.proj_size}"
        return s


class _FloatGates:
    """``x W^T + b`` with the float32 weights (``lq_linear_f32``)."""

    def _gates(self, name: str, x_ptr: int, ldx: int, M: int, K: int, y_ptr: int, ldy: int = 0) -> None:
        from lucid_amd.quantization._device import on_device

        w = on_device(getattr(self, "weight_" + name))
        b = getattr(self, "bias_" + name, None)
        b = on_device(b) if b is not None else None
        N = int(w.shape[0])
        self._alive = (w, b)
        _C.call("lq_linear_f32", x_ptr, ldx, w.data_ptr(), K, b.data_ptr() if b is not None else None, y_ptr,
                ldy or N, M, N, K, None)


class LSTM(_FloatGates, _RNNBase):
    """Multi-layer LSTM (gates i, f, g, o)."""

    def __init__(self, input_size: int, hidden_size: int, num_layers: int = 1, bias: bool = True,
                 batch_first: bool = False, dropout: float = 0.0, bidirectional: bool = False,
                 proj_size: int = 0) -> None:
        super().__init__("LSTM", input_size, hidden_size, num_layers, bias, batch_first, dropout, bidirectional,
                         proj_size)

    def forward(self, input: Tensor, hx: tuple[Tensor, Tensor] | None = None):
        h0, c0 = (None, None) if hx is None else hx
        out, h_n, c_n = self._run(input, h0, c0)
        return out, (h_n, c_n)


class GRU(_FloatGates, _RNNBase):
    """Multi-layer GRU (gates r, z, n)."""

    def __init__(self, input_size: int, hidden_size: int, num_layers: int = 1, bias: bool = True,
                 batch_first: bool = False, dropout: float = 0.0, bidirectional: bool = False) -> None:
        super().__init__("GRU", input_size, hidden_size, num_layers, bias, batch_first, dropout, bidirectional)

    def forward(self, input: Tensor, hx: Tensor | None = None):
        out, h_n, _ = self._run(input, hx, None)
        return out, h_n


class _CellBase(_Recurrent):
    def __init__(self, mode: str, input_size: int, hidden_size: int, bias: bool = True) -> None:
        super().__init__()
        self.mode = mode
        self.input_size, self.hidden_size, self.bias = input_size, hidden_size, bias
        G = _GATES[mode]
        self.weight_ih = Parameter(_init_uniform((G * hidden_size, input_size), hidden_size))
        self.weight_hh = Parameter(_init_uniform((G * hidden_size, hidden_size), hidden_size))
        if bias:
            self.bias_ih = Parameter(_init_uniform((G * hidden_size,), hidden_size))
            self.bias_hh = Parameter(_init_uniform((G * hidden_size,), hidden_size))
        else:
            self.register_parameter("bias_ih", None)
            self.register_parameter("bias_hh", None)

    def _step(self, input: Tensor, hx: Tensor | None, cx: Tensor | None):
        require_gpu(input, type(self).__name__)
        if input.dtype != float32:
            raise TypeError(f"{type(self).__name__}: float32 input expected, got {input.dtype}")
        unbatched = input.ndim == 1
        x = input.reshape(1, input.shape[0]) if unbatched else input
        B, H, G = int(x.shape[0]), self.hidden_size, _GATES[self.mode]
        if int(x.shape[1]) != self.input_size:
            raise ValueError(f"{type(self).__name__}: input size {int(x.shape[1])} != {self.input_size}")
        h = self._state(hx, 0, B)
        c = self._state(cx, 0, B) if self.mode == "LSTM" else None
        gx = empty((B, G * H), float32, "gpu")
        gh = empty((B, G * H), float32, "gpu")
        self._gates("ih", x.data_ptr(), self.input_size, B, self.input_size, gx.data_ptr())
        self._gates("hh", h.data_ptr(), H, B, H, gh.data_ptr())
        _C.call("lq_rnn_cell", _KIND[self.mode], gx.data_ptr(), G * H, gh.data_ptr(), G * H, h.data_ptr(),
                c.data_ptr() if c is not None else None, B, H, h.data_ptr(),
                c.data_ptr() if c is not None else None, None, 0, None)
        if unbatched:
            h = h.reshape(H)
            c = c.reshape(H) if c is not None else None
        return h, c

    def extra_repr(self) -> str:
        return f"{self.input_size}, {self.hidden_size}"


class RNNCell(_FloatGates, _CellBase):
    """Elman cell, ``tanh`` or ``relu`` nonlinearity."""

    def __init__(self, input_size: int, hidden_size: int, bias: bool = True, nonlinearity: str = "tanh") -> None:
        if nonlinearity not in ("tanh", "relu"):
            raise ValueError(f"Unknown nonlinearity {nonlinearity!r}. Select from 'tanh' or 'relu'.")
        super().__init__("RNN_TANH" if nonlinearity == "tanh" else "RNN_RELU", input_size, hidden_size, bias)
        self.nonlinearity = nonlinearity

    def forward(self, input: Tensor, hx: Tensor | None = None) -> Tensor:
        return self._step(input, hx, None)[0]


class LSTMCell(_FloatGates, _CellBase):
    def __init__(self, input_size: int, hidden_size: int, bias: bool = True) -> None:
        super().__init__("LSTM", input_size, hidden_size, bias)

    def forward(self, input: Tensor, hx: tuple[Tensor, Tensor] | None = None):
        h0, c0 = (None, None) if hx is None else hx
        return self._step(input, h0, c0)


class GRUCell(_FloatGates, _CellBase):
    def __init__(self, input_size: int, hidden_size: int, bias: bool = True) -> None:
        super().__init__("GRU", input_size, hidden_size, bias)

    def forward(self, input: Tensor, hx: Tensor | None = None) -> Tensor:
        return self._step(input, hx, None)[0]
