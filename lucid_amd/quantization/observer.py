"""Observers: running range statistics that become ``(scale, zero_point)``.

Names, constructor arguments, buffers (``min_val`` / ``max_val`` seeded ``+inf`` /
``-inf``) and update rules follow lucid/quantization/observer.py:

* ``MinMaxObserver``: ``min_val = minimum(min_val, x.min())`` (observer.py:408-414);
* ``MovingAverageMinMaxObserver``: first batch seeds, then
  ``m + c * (cur - m)`` (observer.py:527-544);
* ``PerChannelMinMaxObserver``: ``amin/amax`` over every axis but ``ch_axis``, the
  scalar seed broadcasting to ``(C,)`` on the first batch (observer.py:672-685);
* ``MovingAveragePerChannelMinMaxObserver`` (observer.py:1031-1048).

Each forward is two device launches (per-block extrema, then a fold into the running
buffers, lucid_amd/csrc/lq_quant.hip): a single read of ``x`` where the reference runs
two full reductions plus 0-d ops.  Running buffers live on the input's device and are
updated in place; the input is returned unchanged.
"""

from __future__ import annotations

import functools
from typing import Any

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, tensor
from lucid_amd.nn.module import Module
from lucid_amd.quantization._device import ocl, require_gpu, workspace
from lucid_amd.quantization._qparams import calculate_qparams
from lucid_amd.quantization._qscheme import (
    QDtype,
    QScheme,
    per_channel_symmetric,
    per_tensor_affine,
    qint8,
    quint8,
)


class ObserverBase(Module):
    """Base of every observer: qscheme / qdtype / ch_axis / eps and buffer alignment."""

    def __init__(self, qscheme: QScheme, qdtype: QDtype, ch_axis: int | None = None,
                 eps: float = 1e-8) -> None:
        super().__init__()
        self.qscheme = qscheme
        self.qdtype = qdtype
        self.ch_axis = ch_axis if qscheme.is_per_channel else None
        self.eps = eps

    def _align_running_buffers(self, ref: Tensor) -> None:
        """Move running buffers to ``ref``'s device; a scalar seed of a per-channel
        observer grows to ``(C,)`` (observer.py:226-246)."""
        ch = None
        if self.ch_axis is not None and ref.ndim > 0:
            ch = ref.shape[self.ch_axis]
        for name, buf in list(self._buffers.items()):
            if buf is None:
                continue
            want = (ch,) if ch is not None and buf.ndim == 0 else buf.shape
            if buf.device != ref.device or tuple(buf.shape) != tuple(want):
                arr = buf.numpy()
                if tuple(arr.shape) != tuple(want):
                    arr = np.ascontiguousarray(np.broadcast_to(arr, want))
                self.register_buffer(name, tensor(arr, device=ref.device))

    def _load_from_state_dict(self, state_dict: dict, prefix: str, local_metadata: dict,
                              strict: bool, missing_keys: list, unexpected_keys: list,
                              error_msgs: list) -> None:
        """A saved buffer of another shape (a per-channel ``(C,)`` into a fresh scalar seed)
        replaces the current one (observer.py:248-281)."""
        for name, cur in list(self._buffers.items()):
            saved = state_dict.get(prefix + name)
            if saved is None or cur is None:
                continue
            if tuple(saved.shape) != tuple(cur.shape):
                self.register_buffer(name, saved.to(cur.device))
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        raise NotImplementedError

    @classmethod
    def with_args(cls, **kwargs: Any) -> functools.partial:
        """A constructor recipe for a ``QConfig`` (observer.py:288-295)."""
        return functools.partial(cls, **kwargs)


def _fold_minmax(obs: ObserverBase, x: Tensor, mode: int, c: float) -> None:
    require_gpu(x, type(obs).__name__)
    if x.dtype != np.float32:
        raise TypeError(f"{type(obs).__name__}: expected float32 input, got {x.dtype}")
    obs._align_running_buffers(x)
    n = x.numel()
    L = _C.lib()
    ws_bytes = L.lq_minmax_workspace_size(n)
    _C.call("lq_minmax_f32", x.data_ptr() if n else None, n, obs.min_val.data_ptr(),
            obs.max_val.data_ptr(), mode, float(np.float32(c)), workspace.get(ws_bytes), ws_bytes,
            None)


def _fold_minmax_per_channel(obs: ObserverBase, x: Tensor, mode: int, c: float) -> None:
    require_gpu(x, type(obs).__name__)
    if x.dtype != np.float32:
        raise TypeError(f"{type(obs).__name__}: expected float32 input, got {x.dtype}")
    axis = obs.ch_axis if obs.ch_axis is not None else 0
    obs._align_running_buffers(x)
    outer, C, inner = ocl(x.shape, axis)
    L = _C.lib()
    ws_bytes = L.lq_minmax_per_channel_workspace_size(outer, C, inner)
    _C.call("lq_minmax_per_channel_f32", x.data_ptr() if x.numel() else None, outer, C, inner,
            obs.min_val.data_ptr(), obs.max_val.data_ptr(), mode, float(np.float32(c)),
            workspace.get(ws_bytes), ws_bytes, None)


class MinMaxObserver(ObserverBase):
    """Cumulative per-tensor range."""

    def __init__(self, qscheme: QScheme = per_tensor_affine, qdtype: QDtype = quint8,
                 eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, None, eps)
        self.register_buffer("min_val", tensor(np.float32(np.inf)))
        self.register_buffer("max_val", tensor(np.float32(-np.inf)))

    def forward(self, x: Tensor) -> Tensor:
        _fold_minmax(self, x, _C.OBS_MINMAX, 0.0)
        return x

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        return calculate_qparams(self.min_val, self.max_val, self.qscheme, self.qdtype, self.eps)


class MovingAverageMinMaxObserver(MinMaxObserver):
    """EMA of the per-tensor range: ``m + c * (cur - m)`` after a seeding first batch."""

    def __init__(self, qscheme: QScheme = per_tensor_affine, qdtype: QDtype = quint8,
                 averaging_constant: float = 0.01, eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, eps)
        self.averaging_constant = averaging_constant

    def forward(self, x: Tensor) -> Tensor:
        _fold_minmax(self, x, _C.OBS_EMA, self.averaging_constant)
        return x


class PerChannelMinMaxObserver(ObserverBase):
    """Cumulative per-channel range along ``ch_axis``."""

    def __init__(self, ch_axis: int = 0, qscheme: QScheme = per_channel_symmetric,
                 qdtype: QDtype = qint8, eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, ch_axis, eps)
        self.register_buffer("min_val", tensor(np.float32(np.inf)))
        self.register_buffer("max_val", tensor(np.float32(-np.inf)))

    def _align_running_buffers(self, ref: Tensor) -> None:
        # The reduction axis is ch_axis (0 when the scheme is per-tensor), as in forward.
        if self.ch_axis is None:
            saved = self.ch_axis
            self.ch_axis = 0
            try:
                super()._align_running_buffers(ref)
            finally:
                self.ch_axis = saved
        else:
            super()._align_running_buffers(ref)

    def forward(self, x: Tensor) -> Tensor:
        _fold_minmax_per_channel(self, x, _C.OBS_MINMAX, 0.0)
        return x

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        return calculate_qparams(self.min_val, self.max_val, self.qscheme, self.qdtype, self.eps)


class MovingAveragePerChannelMinMaxObserver(PerChannelMinMaxObserver):
    """Per-channel EMA; the first batch (all of ``min_val`` infinite) seeds."""

    def __init__(self, ch_axis: int = 0, qscheme: QScheme = per_channel_symmetric,
                 qdtype: QDtype = qint8, averaging_constant: float = 0.01,
                 eps: float = 1e-8) -> None:
        super().__init__(ch_axis, qscheme, qdtype, eps)
        self.averaging_constant = averaging_constant

    def forward(self, x: Tensor) -> Tensor:
        _fold_minmax_per_channel(self, x, _C.OBS_EMA, self.averaging_constant)
        return x


class HistogramObserver(ObserverBase):
    """Lucid's default static activation observer (observer.py:692-926).

    Not part of this backend yet: its L2 clip-range search over a 2048-bin histogram
    is a later addition.  Pin ``MinMaxObserver`` (or a moving-average observer) as the
    activation observer of a ``QConfig`` instead.
    """

    def __init__(self, bins: int = 2048, qscheme: QScheme = per_tensor_affine,
                 qdtype: QDtype = quint8, eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, None, eps)
        self.bins = bins
        self.register_buffer("min_val", tensor(np.float32(np.inf)))
        self.register_buffer("max_val", tensor(np.float32(-np.inf)))
        self.register_buffer("histogram", tensor(np.zeros(bins, np.float32)))

    def forward(self, x: Tensor) -> Tensor:
        raise NotImplementedError(
            "HistogramObserver is not implemented on the HIP backend; use "
            "MinMaxObserver / MovingAverageMinMaxObserver as the activation observer"
        )

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        raise NotImplementedError("HistogramObserver is not implemented on the HIP backend")


class FixedQParamsObserver(ObserverBase):
    """Fixed ``(scale, zero_point)``; identity forward (observer.py:1053-1166)."""

    def __init__(self, scale: float, zero_point: int, qscheme: QScheme = per_tensor_affine,
                 qdtype: QDtype = quint8, eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, None, eps)
        self.register_buffer("scale", tensor(np.float32(float(scale))))
        self.register_buffer("zero_point", tensor(np.float32(float(zero_point))))

    def forward(self, x: Tensor) -> Tensor:
        return x

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        return self.scale, self.zero_point


class PlaceholderObserver(ObserverBase):
    """Metadata only; ``calculate_qparams`` raises (observer.py:1168-1262)."""

    def __init__(self, qscheme: QScheme = per_tensor_affine, qdtype: QDtype = quint8,
                 eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, None, eps)

    def forward(self, x: Tensor) -> Tensor:
        return x

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        raise RuntimeError(
            f"{type(self).__name__} collects no statistics; qparams are computed "
            "at runtime (dynamic quantization) or supplied elsewhere."
        )


class NoopObserver(PlaceholderObserver):
    """A placeholder that marks a tensor as not quantized."""
