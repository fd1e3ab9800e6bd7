"""Replay a module forward as one HIP graph.

:class:`CapturedForward` runs a forward once while recording every C-ABI call it makes
(``_C.call``) and keeping alive every device buffer allocated meanwhile, then captures the
recorded launches, in order, into a HIP graph on a stream of its own.  Each replay runs the
same kernels on the same buffers: the inputs given at construction are the graph's inputs
(copy new data into them with :meth:`CapturedForward.load`), and the forward's result tensor
is refilled in place.  Python module dispatch and allocation leave the replayed path: the
launches are those of the eager forward, so the results are its bits.

Lucid runs modules eagerly (no graph form); this is the device-side counterpart of a static
inference loop.  Requirements, checked while recording: every call is a device launch whose
last argument is the stream, issued on the default stream (the replay substitutes its own),
and no call copies between host and device or synchronizes.  The forward's scratch comes
from a private workspace held by the capture, so eager calls made between replays do not
share it; replays and eager work on other streams are ordered by the caller (synchronize).
"""

from __future__ import annotations

import ctypes
import os
import re

from lucid_amd import _C
from lucid_amd import _tensor as _T

_HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "lq_api.h")
_stream_last: set | None = None


def _stream_last_entries() -> set:
    """Entry points whose last parameter is ``void* stream`` (from the C header)."""
    global _stream_last
    if _stream_last is None:
        with open(_HEADER) as f:
            text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
        found = set()
        for m in re.finditer(r"\bint\s+(lq_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
            params = [p.strip() for p in m.group(2).split(",")]
            if params and re.fullmatch(r"void\s*\*\s*stream", params[-1]):
                found.add(m.group(1))
        _stream_last = found
    return _stream_last


class CaptureError(RuntimeError):
    """The forward made a call a graph cannot replay."""


_UNREPLAYABLE = {"lq_memcpy_h2d", "lq_memcpy_d2h", "lq_stream_synchronize", "lq_device_synchronize",
                 "lq_event_synchronize", "lq_graph_begin_capture", "lq_graph_end_capture", "lq_graph_launch"}


class CapturedForward:
    """``fn(*inputs)`` recorded once and captured as a HIP graph (see the module docstring).

    ``warmup`` eager calls come first, so one-time work (weight packing, device copies of
    buffers, plan caches) stays out of the recording."""

    def __init__(self, fn, *inputs, warmup: int = 2) -> None:
        from lucid_amd.quantization._device import workspace

        for _ in range(warmup):
            fn(*inputs)
        _C.synchronize()
        local = workspace._local
        saved_ws = getattr(local, "buf", None)
        local.buf = None  # the recorded forward allocates its own scratch
        held: list = []
        calls: list = []
        _T._held, _C._recording = held, calls
        try:
            out = fn(*inputs)
            # a code-backed result materializes its float view once and keeps it: do that
            # inside the recording, so every replay refreshes it from the new codes
            for t in (out if isinstance(out, (tuple, list)) else (out,)):
                if isinstance(t, _T.Tensor) and t.is_code_backed and t._buf is None and t.device == "gpu":
                    t.data_ptr()
        finally:
            _T._held, _C._recording = None, None
            private_ws = getattr(local, "buf", None)
            local.buf = saved_ws
        _C.synchronize()
        stream_last = _stream_last_entries()
        for name, args in calls:
            if name in _UNREPLAYABLE:
                raise CaptureError(f"CapturedForward: the forward calls {name}, which a graph cannot replay")
            if name not in stream_last:
                raise CaptureError(f"CapturedForward: {name} takes no stream argument")
            if args[-1] is not None:
                raise CaptureError(f"CapturedForward: {name} was issued on a stream of its own")
        self.fn, self.inputs, self.output = fn, inputs, out
        self.calls = calls
        self._held = held + ([private_ws] if private_ws is not None else [])
        self.stream = ctypes.c_void_p()
        _C.call("lq_stream_create", ctypes.byref(self.stream))
        self.exe = None
        _C.call("lq_graph_begin_capture", self.stream)
        try:
            for name, args in calls:
                _C.call(name, *args[:-1], self.stream)
        finally:
            exe = ctypes.c_void_p()
            _C.call("lq_graph_end_capture", self.stream, ctypes.byref(exe))
        self.exe = exe

    @property
    def launches(self) -> int:
        return len(self.calls)

    def load(self, *arrays) -> None:
        """Copy host arrays into the captured inputs (same shapes and dtypes)."""
        import numpy as np

        for t, a in zip(self.inputs, arrays):
            a = np.ascontiguousarray(a, dtype=t.dtype)
            if tuple(a.shape) != tuple(t.shape):
                raise ValueError(f"CapturedForward.load: shape {a.shape} for an input of shape {tuple(t.shape)}")
            _C.call("lq_memcpy_h2d", t.data_ptr(), a.ctypes.data, a.nbytes, self.stream)
        _C.call("lq_stream_synchronize", self.stream)

    def replay(self):
        """Launch the graph on the capture's stream and return the forward's result tensor
        (refilled when the stream reaches the end of the replay)."""
        _C.call("lq_graph_launch", self.exe, self.stream)
        return self.output

    def synchronize(self) -> None:
        _C.call("lq_stream_synchronize", self.stream)

    def __call__(self):
        out = self.replay()
        self.synchronize()
        return out

    def __del__(self) -> None:
        if _C._lib is None:
            return
        if getattr(self, "exe", None) is not None:
            _C._lib.lq_graph_destroy(self.exe)
            self.exe = None
        if getattr(self, "stream", None) is not None and self.stream.value:
            _C._lib.lq_stream_destroy(self.stream)
            self.stream = None
