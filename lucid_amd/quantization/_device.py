"""Helpers shared by the quantization ops: device checks, qparam marshalling, workspace."""

from __future__ import annotations

import threading
from typing import Any

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, _DeviceBuffer, float32, tensor

# numpy storage dtype -> backend code type
CODE_TYPE = {
    np.dtype(np.int8): _C.I8,
    np.dtype(np.uint8): _C.U8,
    np.dtype(np.int16): _C.I16,
    np.dtype(np.int32): _C.I32,
}


def require_gpu(x: Tensor, op: str) -> None:
    """Device ops run on the GPU only (as Lucid's engine.quantized requires Metal tensors,
    lucid/_C/ops/quantized/QuantizedMatmul.cpp:41-49)."""
    if not isinstance(x, Tensor):
        raise TypeError(f"{op}: expected a Tensor, got {type(x).__name__}")
    if x.device != "gpu":
        raise _C.LucidError(
            f"{op}: quantized ops of this backend run on GPU tensors; move the input with "
            f".to('gpu') (got a {x.device} tensor)"
        )


def on_device(p: Tensor, device: str = "gpu") -> Tensor:
    """A qparam tensor on the data's device (quantize() moves qparams, _functional.py:186-189)."""
    if p.device != device:
        p = p.to(device)
    if p.dtype != float32:
        p = tensor(p.numpy().astype(np.float32), device=device)
    return p


def scalar_tensor(value: Any, device: str = "gpu") -> Tensor:
    """A Python number as a 0-d float32 tensor (``full([], float(x), F32)``,
    lucid/_dispatch.py:154-171)."""
    return tensor(np.float32(float(value)), device=device)


def ocl(shape: tuple[int, ...], ch_axis: int) -> tuple[int, int, int]:
    """[outer, C, inner] view of ``shape`` around ``ch_axis`` (the reshape that
    _reshape_for_channel broadcasts along, lucid/quantization/_functional.py:47-56)."""
    nd = len(shape)
    if nd == 0:
        raise ValueError("per-channel op on a 0-d tensor")
    ax = ch_axis + nd if ch_axis < 0 else ch_axis
    if not 0 <= ax < nd:
        raise ValueError(f"ch_axis {ch_axis} out of range for {nd}-d input")
    outer = int(np.prod(shape[:ax], dtype=np.int64))
    inner = int(np.prod(shape[ax + 1:], dtype=np.int64))
    return outer, int(shape[ax]), inner


class _Workspace:
    """One growing device scratch buffer per thread (kernels on one stream reuse it in order)."""

    def __init__(self) -> None:
        self._local = threading.local()

    def get(self, nbytes: int) -> int:
        buf = getattr(self._local, "buf", None)
        if buf is None or buf.nbytes < nbytes:
            buf = _DeviceBuffer(max(int(nbytes), 256))
            self._local.buf = buf
        return buf.ptr


workspace = _Workspace()
