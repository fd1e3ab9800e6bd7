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
import math
from typing import Any

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, tensor
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
    """Per-tensor observer that keeps a value histogram and picks the clip range with the
    least expected L2 quantization error (observer.py:692-926); Lucid's default static
    activation observer.

    Buffers ``min_val`` / ``max_val`` (running support, seeded ``+inf`` / ``-inf``) and
    ``histogram`` (``bins`` float32 counts).  ``forward`` reads the batch range back (as
    Lucid's ``.item()`` calls do), widens the running range, moves the stored counts onto
    the wider bins when it grows (``lq_hist_rebin_f32``) and adds the batch's counts
    (``lq_histc_f32``) -- the counting runs on the GPU in one pass over ``x``.
    ``calculate_qparams`` runs the reference's coarse clip search on the host over the
    ``bins`` counts (a data-dependent scan of a few thousand numbers, observer.py:872-926,
    where Lucid runs it too) and reduces the winning range with ``calculate_qparams``.
    """

    _QUANTILES = (0.0, 1e-5, 1e-4, 1e-3, 5e-3, 1e-2)

    def __init__(self, bins: int = 2048, qscheme: QScheme = per_tensor_affine,
                 qdtype: QDtype = quint8, eps: float = 1e-8) -> None:
        super().__init__(qscheme, qdtype, None, eps)
        self.bins = bins
        self.register_buffer("min_val", tensor(np.float32(np.inf)))
        self.register_buffer("max_val", tensor(np.float32(-np.inf)))
        self.register_buffer("histogram", tensor(np.zeros(bins, np.float32)))

    def _batch_range(self, x: Tensor) -> tuple[float, float]:
        """``x.min()``, ``x.max()`` (NaN-propagating) read back to the host."""
        n = x.numel()
        ext = tensor(np.array([np.inf, -np.inf], np.float32), device="gpu")
        L = _C.lib()
        ws_bytes = L.lq_minmax_workspace_size(n)
        _C.call("lq_minmax_f32", x.data_ptr(), n, ext.data_ptr(), ext.data_ptr() + 4, _C.OBS_REPLACE,
                0.0, workspace.get(ws_bytes), ws_bytes, None)
        lo, hi = ext.numpy().tolist()
        return float(lo), float(hi)

    def _histc_range(self, x_lo: float, x_hi: float, lo: float, hi: float) -> tuple[float, float]:
        """The range histc counts over (lucid/_ops/_adapters.py:1266-1276)."""
        if lo > hi:
            raise ValueError(f"histc: max must be at least min, got [{lo}, {hi}]")
        if lo == hi:
            lo, hi = x_lo, x_hi
        if not (math.isfinite(lo) and math.isfinite(hi)):
            raise ValueError(f"histc: range of [{lo}, {hi}] is not finite")
        if lo == hi:
            lo, hi = lo - 1.0, hi + 1.0
        return lo, hi

    def forward(self, x: Tensor) -> Tensor:
        require_gpu(x, type(self).__name__)
        if x.dtype != np.float32:
            raise TypeError(f"{type(self).__name__}: expected float32 input, got {x.dtype}")
        n = x.numel()
        if n == 0:
            raise ValueError("HistogramObserver: an empty batch has no range")
        self._align_running_buffers(x)
        if self.histogram.numel() != self.bins:
            raise ValueError(f"HistogramObserver: histogram buffer has {self.histogram.numel()} "
                             f"bins, expected {self.bins}")
        cur_min, cur_max = self._batch_range(x)
        old_min, old_max = float(self.min_val.item()), float(self.max_val.item())
        first = old_min == math.inf
        if first:
            new_min, new_max = cur_min, cur_max
        else:
            new_min, new_max = min(old_min, cur_min), max(old_max, cur_max)
        lo, hi = self._histc_range(cur_min, cur_max, new_min, new_max)
        L = _C.lib()
        ws_bytes = L.lq_histc_workspace_size(self.bins)
        hist = self.histogram
        if not first and not (new_min == old_min and new_max == old_max):
            # the stored counts move onto the wider bins first (observer.py:865)
            hist = empty((self.bins,), np.float32, "gpu")
            _C.call("lq_hist_rebin_f32", self.histogram.data_ptr(), self.bins, float(np.float32(old_min)),
                    float(np.float32((old_max - old_min) / self.bins)), float(np.float32(new_min)),
                    float(np.float32((new_max - new_min) / self.bins)), hist.data_ptr(), None)
        _C.call("lq_histc_f32", x.data_ptr(), n, self.bins, lo, hi, 0 if first else 1, hist.data_ptr(),
                workspace.get(ws_bytes), ws_bytes, None)
        if hist is not self.histogram:
            self.histogram.copy_(hist)
        self.min_val.copy_(tensor(np.float32(new_min), device="gpu"))
        self.max_val.copy_(tensor(np.float32(new_max), device="gpu"))
        return x

    def _search_clip_range(self) -> tuple[float, float]:
        """The candidate clip range with the least clip-plus-rounding error
        (observer.py:872-901), scanned in double precision in source order."""
        lo, hi = float(self.min_val.item()), float(self.max_val.item())
        counts = [float(c) for c in self.histogram.numpy().tolist()]
        total = sum(counts)
        if total <= 0.0 or hi <= lo:
            return lo, hi
        bins = self.bins
        width = (hi - lo) / bins
        centers = [lo + (i + 0.5) * width for i in range(bins)]
        levels = self.qdtype.quant_max - self.qdtype.quant_min
        best_err, best = math.inf, (lo, hi)
        for frac in self._QUANTILES:
            cmin = _quantile_from_hist(counts, centers, frac)
            cmax = _quantile_from_hist(counts, centers, 1.0 - frac)
            if cmax <= cmin:
                continue
            step = (cmax - cmin) / max(levels, 1)
            err = 0.0
            for c, k in zip(centers, counts):
                if k == 0.0:
                    continue
                cc = cmin if c < cmin else (cmax if c > cmax else c)
                err += k * ((c - cc) ** 2 + (step * step) / 12.0)
            if err < best_err:
                best_err, best = err, (cmin, cmax)
        return best

    def calculate_qparams(self) -> tuple[Tensor, Tensor]:
        new_min, new_max = self._search_clip_range()
        return calculate_qparams(float(new_min), float(new_max), self.qscheme, self.qdtype, self.eps)


def _quantile_from_hist(counts: list[float], centers: list[float], q: float) -> float:
    """The bin center where the cumulative count first reaches ``q`` of the total
    (observer.py:915-926)."""
    total = sum(counts)
    if total <= 0:
        return centers[0]
    target = q * total
    acc = 0.0
    for c, k in zip(centers, counts):
        acc += k
        if acc >= target:
            return c
    return centers[-1]


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
