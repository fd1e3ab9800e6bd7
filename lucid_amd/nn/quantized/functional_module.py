"""Quantizable merges -- ``add`` / ``mul`` / ``add_relu`` / ``cat`` / ``add_scalar`` /
``mul_scalar`` (lucid/nn/quantized/functional_module.py:23-235).

A residual network quantizes end to end only if each merge output is observed and then
requantized onto one grid.  ``FloatFunctional`` is the calibration-time module a model calls
instead of ``x + y`` / ``cat``; ``prepare`` attaches an observer to it and ``convert`` swaps
it for ``QFunctional``, which snaps every merge result onto the calibrated
``(scale, zero_point)``.

Both run ``lq_qmerge``: one kernel that reads each operand as float32 or, when the operand is
a code-backed activation (the output of a quantized layer), straight from its integer codes
and grid; ``QFunctional`` writes codes, so its result is code-backed too and the next
quantized layer consumes them without a float round trip.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import QuantSource, Tensor, empty
from lucid_amd.nn.module import Module
from lucid_amd.nn.quantized._utils import _QuantizedGridModule, activation_qparams
from lucid_amd.quantization._device import on_device, require_gpu
from lucid_amd.quantization._qscheme import QDtype, quint8


def _operand(x: Tensor, op: str) -> tuple[int, int, int | None, int | None]:
    """(pointer, element type, scale pointer, zero-point pointer) of a merge operand: the
    codes of a code-backed activation, else its float32 storage."""
    require_gpu(x, op)
    q = x.quant_source
    if q is not None and q.code_type in (_C.I8, _C.U8, _C.I16, _C.U8S8):
        return q.codes.data_ptr(), q.code_type, q.scale.data_ptr(), q.zero_point.data_ptr()
    if x.dtype != np.float32:
        raise TypeError(f"{op}: expected float32 tensors, got {x.dtype}")
    return x.data_ptr(), _C.F32, None, None


def _grid_codes(qmin: int, qmax: int) -> tuple[int, type] | None:
    """The code storage of an output grid (the same choice as fake_quantize_to_codes)."""
    if qmin >= -128 and qmax <= 127:
        return _C.I8, np.int8
    if qmin >= 0 and qmax <= 255:
        return _C.U8S8, np.int8
    if qmin >= -32768 and qmax <= 32767:
        return _C.I16, np.int16
    return None


class _MergeBase(Module):
    """The merge surface shared by the float and the quantized module."""

    def _merge(self, op: int, a: Tensor, b: Tensor | None, scalar: float, relu: bool, name: str) -> Tensor:
        pa = _operand(a, name)
        pb = (0, _C.F32, None, None)
        if b is not None:
            if tuple(a.shape) != tuple(b.shape):
                raise ValueError(f"{name}: operand shapes differ ({a.shape} vs {b.shape}); "
                                 "broadcasting merges are not supported")
            pb = _operand(b, name)
        n = a.numel()
        return self._post(self._emit(op, pa, pb, scalar, relu, 1, n, n, a.shape))

    def _emit(self, op, pa, pb, scalar, relu, rows, cols, ld, shape, out=None, out_off=0) -> Tensor:
        """Run one lq_qmerge into ``out`` (allocated when None) at element offset ``out_off``."""
        raise NotImplementedError

    def _post(self, y: Tensor) -> Tensor:
        """What happens to a finished merge result (observation, for the float module)."""
        return y

    def add(self, x: Tensor, y: Tensor) -> Tensor:
        """``x + y`` (a residual skip-add)."""
        return self._merge(_C.MERGE_ADD, x, y, 0.0, False, "add")

    def mul(self, x: Tensor, y: Tensor) -> Tensor:
        """``x * y``."""
        return self._merge(_C.MERGE_MUL, x, y, 0.0, False, "mul")

    def add_relu(self, x: Tensor, y: Tensor) -> Tensor:
        """``relu(x + y)``, the fused residual add of a ResNet block."""
        return self._merge(_C.MERGE_ADD, x, y, 0.0, True, "add_relu")

    def add_scalar(self, x: Tensor, scalar: float) -> Tensor:
        """``x + scalar`` (the scalar rounded to float32, as a 0-d operand is)."""
        return self._merge(_C.MERGE_ADD_SCALAR, x, None, float(np.float32(scalar)), False, "add_scalar")

    def mul_scalar(self, x: Tensor, scalar: float) -> Tensor:
        """``x * scalar``."""
        return self._merge(_C.MERGE_MUL_SCALAR, x, None, float(np.float32(scalar)), False, "mul_scalar")

    def cat(self, tensors: Sequence[Tensor], dim: int = 0) -> Tensor:
        """Concatenation along ``dim``: each input is written into its slice of the result."""
        tensors = list(tensors)
        if not tensors:
            raise ValueError("cat: expected a non-empty list of tensors")
        nd = tensors[0].ndim
        d = dim + nd if dim < 0 else dim
        if not 0 <= d < nd:
            raise IndexError(f"cat: dim {dim} out of range for {nd}-d tensors")
        base = tuple(tensors[0].shape)
        for t in tensors:
            if t.ndim != nd or tuple(t.shape[:d]) != base[:d] or tuple(t.shape[d + 1:]) != base[d + 1:]:
                raise ValueError(f"cat: shapes {base} and {tuple(t.shape)} differ outside dim {d}")
        outer = int(np.prod(base[:d], dtype=np.int64))
        inner = int(np.prod(base[d + 1:], dtype=np.int64))
        total = sum(int(t.shape[d]) for t in tensors)
        shape = base[:d] + (total,) + base[d + 1:]
        out, off = None, 0
        for t in tensors:
            cols = int(t.shape[d]) * inner
            out = self._emit(_C.MERGE_COPY, _operand(t, "cat"), (0, _C.F32, None, None), 0.0, False, outer,
                             cols, total * inner, shape, out=out, out_off=off * inner)
            off += int(t.shape[d])
        return self._post(out)


class FloatFunctional(_MergeBase):
    """Float merges whose results ``prepare`` observes (functional_module.py:23-120).

    Before ``prepare`` every method is the plain float op; afterwards each result also feeds
    ``activation_post_process``.  One instance per merge site.
    """

    def _emit(self, op, pa, pb, scalar, relu, rows, cols, ld, shape, out=None, out_off=0) -> Tensor:
        y = out if out is not None else empty(shape, np.float32, "gpu")
        if cols and rows:
            _C.call("lq_qmerge", op, pa[0], pa[1], pa[2], pa[3], pb[0], pb[1], pb[2], pb[3], scalar, rows, cols, ld,
                    None, None, 0, 0, _C.EPI_RELU if relu else 0, _C.F32, y.data_ptr() + 4 * out_off, None)
        return y

    def _post(self, y: Tensor) -> Tensor:
        """Feed the result to the attached observer (identity before ``prepare``)."""
        app = getattr(self, "activation_post_process", None)
        return app(y) if app is not None else y

    def forward(self, *args, **kwargs):
        raise RuntimeError("FloatFunctional is not called directly: use add / mul / add_relu / cat / "
                           "add_scalar / mul_scalar")


class QFunctional(_QuantizedGridModule, _MergeBase):
    """Quantized merges: every result fake-quantized onto one calibrated grid
    (functional_module.py:125-235); ``add_relu`` applies the ReLU before the grid.  Buffers
    ``scale`` / ``zero_point`` as Lucid's.  The result is code-backed."""

    def __init__(self, scale: Tensor, zero_point: Tensor, qdtype: QDtype = quint8) -> None:
        super().__init__(scale, zero_point, qdtype)

    def _emit(self, op, pa, pb, scalar, relu, rows, cols, ld, shape, out=None, out_off=0) -> Tensor:
        qmin, qmax = self.qdtype.quant_min, self.qdtype.quant_max
        grid = _grid_codes(qmin, qmax)
        if grid is None:
            raise ValueError(f"QFunctional: a [{qmin}, {qmax}] grid does not fit 16-bit codes")
        code_type, dt = grid
        s, z = on_device(self.scale), on_device(self.zero_point)
        if out is None:
            codes = empty(shape, dt, "gpu")
            out = Tensor._code_backed(QuantSource(codes, code_type, s, z, qmin, qmax), shape)
        codes = out.quant_source.codes
        if cols and rows:
            _C.call("lq_qmerge", op, pa[0], pa[1], pa[2], pa[3], pb[0], pb[1], pb[2], pb[3], scalar, rows, cols, ld,
                    s.data_ptr(), z.data_ptr(), qmin, qmax, _C.EPI_RELU if relu else 0, code_type,
                    codes.data_ptr() + np.dtype(dt).itemsize * out_off, None)
        return out

    def forward(self, *args, **kwargs):
        raise RuntimeError("QFunctional is not called directly: use add / mul / add_relu / cat / "
                           "add_scalar / mul_scalar")

    @classmethod
    def from_float(cls, mod: Module) -> "QFunctional":
        """From a calibrated ``FloatFunctional`` (its observer's qparams)."""
        scale, zero_point, qdtype = activation_qparams(mod)
        return cls(scale, zero_point, qdtype)
