"""Minimal tensor of the HIP backend: host (numpy) or device (HBM) storage.

Lucid's quantized path needs only a small part of ``lucid.Tensor``: shape,
dtype, device, ``.to(device)``, ``.numpy()``, ``.item()``, ``reshape`` and
buffer bookkeeping for ``state_dict``.  This class provides exactly that.  Device
memory comes from the backend's caching allocator (``lq_malloc``/``lq_free``);
there is no arithmetic on this class -- compute goes through the quantization
ops, which call the HIP kernels.

A device float tensor may be *code-backed*: produced by a fake-quantize on a
known grid, it carries the integer codes and ``(scale, zero_point)`` instead of
float storage.  Its float values are ``fl32(fl32(code - zero_point) * scale)``,
bit-identical to the fake-quantize output, and are materialised (one dequantize
launch) only when read as floats.  Quantized modules consume the codes directly,
which is how an int8 GEMM can sit behind Lucid's float-in/float-out sidecar
modules (lucid/nn/quantized/linear.py:206-215).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any, Sequence

import numpy as np

from lucid_amd import _C

float32 = np.dtype(np.float32)
float16 = np.dtype(np.float16)
float64 = np.dtype(np.float64)
int8 = np.dtype(np.int8)
uint8 = np.dtype(np.uint8)
int16 = np.dtype(np.int16)
int32 = np.dtype(np.int32)
int64 = np.dtype(np.int64)
uint32 = np.dtype(np.uint32)
bool_ = np.dtype(np.bool_)
# bfloat16 (Lucid's BF16, lucid/_C/core/Dtype.h:63-80): numpy has no such type, so host arrays
# hold the 16-bit patterns in a one-field structured dtype, distinct from uint16 / float16.
# bf16_from_f32 / bf16_to_f32 convert; a device tensor converts with Tensor.to(dtype=...).
bfloat16 = np.dtype([("bfloat16", "<u2")])
FLOAT_TYPE_CODE = {float32: _C.F32, float16: _C.F16, bfloat16: _C.BF16}  # element-type codes


def bf16_from_f32(a: Any) -> np.ndarray:
    """float32 values -> bfloat16 array, round to nearest even (NaN stays a quiet NaN)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.view(bfloat16)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    """bfloat16 array -> float32 (exact)."""
    bits = np.ascontiguousarray(a).view(np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _host_astype(arr: np.ndarray, dt: np.dtype) -> np.ndarray:
    dt = np.dtype(dt)
    if arr.dtype == dt:
        return arr
    if dt == bfloat16:
        return bf16_from_f32(arr if arr.dtype != bfloat16 else bf16_to_f32(arr))
    if arr.dtype == bfloat16:
        return bf16_to_f32(arr).astype(dt)
    return arr.astype(dt)

dtype = np.dtype

_DEVICE_ALIASES = {"cpu": "cpu", "gpu": "gpu", "hip": "gpu", "metal": "gpu"}


def normalize_device(device: Any) -> str:
    if device is None:
        return "cpu"
    d = str(device).split(":")[0].lower()
    if d not in _DEVICE_ALIASES:
        raise ValueError(f"unknown device {device!r} (expected 'cpu' or 'gpu')")
    return _DEVICE_ALIASES[d]


_held: list | None = None  # every buffer allocated while a capture records (lucid_amd.graphs)


class _DeviceBuffer:
    """An ``lq_malloc`` allocation, returned to the cache when collected."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes: int) -> None:
        p = ctypes.c_void_p()
        _C.check(_C.lib().lq_malloc(ctypes.byref(p), max(int(nbytes), 1)), "lq_malloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)
        if _held is not None:
            _held.append(self)

    def __del__(self) -> None:
        ptr = getattr(self, "ptr", None)
        if ptr and _C._lib is not None:
            _C._lib.lq_free(ptr)
            self.ptr = None


@dataclass
class QuantSource:
    """Integer codes behind a code-backed float tensor (see module docstring)."""

    codes: "Tensor"  # device integer tensor, same shape as the float tensor
    code_type: int  # _C code dtype of `codes` (I8, U8, I16, U8S8, ...)
    scale: "Tensor"  # 0-d float32 device tensor
    zero_point: "Tensor"  # 0-d float32 device tensor (integer valued)
    quant_min: int
    quant_max: int


class Tensor:
    __slots__ = ("_host", "_buf", "_offset", "_shape", "_dtype", "_device", "_qsrc",
                 "requires_grad", "__weakref__")

    def __init__(self) -> None:  # use the factories
        self._host: np.ndarray | None = None
        self._buf: _DeviceBuffer | None = None
        self._offset = 0
        self._shape: tuple[int, ...] = ()
        self._dtype = float32
        self._device = "cpu"
        self._qsrc: QuantSource | None = None
        self.requires_grad = False

    # ------------------------------------------------------------ construction
    @classmethod
    def _from_numpy(cls, arr: np.ndarray, device: str = "cpu") -> "Tensor":
        arr = np.asarray(arr, order="C")  # keeps 0-d arrays 0-d (ascontiguousarray does not)
        t = cls()
        t._shape = tuple(int(s) for s in arr.shape)
        t._dtype = arr.dtype
        if device == "cpu":
            t._host = arr.copy()
            t._device = "cpu"
        else:
            t._device = "gpu"
            t._buf = _DeviceBuffer(arr.nbytes)
            _C.call("lq_memcpy_h2d", t._buf.ptr, arr.ctypes.data, arr.nbytes, None)
        return t

    @classmethod
    def _empty(cls, shape: Sequence[int], dt: np.dtype, device: str) -> "Tensor":
        t = cls()
        t._shape = tuple(int(s) for s in shape)
        t._dtype = np.dtype(dt)
        if device == "cpu":
            t._host = np.empty(t._shape, t._dtype)
            t._device = "cpu"
        else:
            t._device = "gpu"
            t._buf = _DeviceBuffer(t.nbytes)
        return t

    @classmethod
    def _element_view(cls, base: "Tensor", index: int) -> "Tensor":
        """A 0-d tensor sharing element ``index`` of a flat device tensor's storage."""
        if base._device != "gpu" or base._buf is None or not 0 <= index < base.numel():
            raise ValueError("_element_view: a materialized device tensor and an index in range")
        t = cls()
        t._shape = ()
        t._dtype = base._dtype
        t._device = "gpu"
        t._buf = base._buf
        t._offset = base._offset + index * base._dtype.itemsize
        return t

    @classmethod
    def _code_backed(cls, q: QuantSource, shape: Sequence[int]) -> "Tensor":
        t = cls()
        t._shape = tuple(int(s) for s in shape)
        t._dtype = float32
        t._device = "gpu"
        t._qsrc = q
        return t

    # ----------------------------------------------------------------- metadata
    @property
    def shape(self) -> tuple[int, ...]:
        return self._shape

    @property
    def dtype(self) -> np.dtype:
        return self._dtype

    @property
    def device(self) -> str:
        return self._device

    @property
    def ndim(self) -> int:
        return len(self._shape)

    def dim(self) -> int:
        return len(self._shape)

    def numel(self) -> int:
        return math.prod(self._shape)

    @property
    def size(self) -> int:
        return self.numel()

    @property
    def nbytes(self) -> int:
        return self.numel() * self._dtype.itemsize

    @property
    def is_code_backed(self) -> bool:
        return self._qsrc is not None

    @property
    def quant_source(self) -> QuantSource | None:
        return self._qsrc

    def data_ptr(self) -> int:
        """Device address of the float/integer storage (materialising codes if needed)."""
        if self._device != "gpu":
            raise _C.LucidError("data_ptr() of a CPU tensor; move it with .to('gpu')")
        if self._buf is None:
            self._materialize()
        return self._buf.ptr + self._offset

    def _materialize(self) -> None:
        q = self._qsrc
        assert q is not None
        self._buf = _DeviceBuffer(self.nbytes)
        self._offset = 0
        _C.call("lq_dequantize_per_tensor", q.codes.data_ptr(), q.code_type, self._buf.ptr, _C.F32,
                self.numel(), q.scale.data_ptr(), q.zero_point.data_ptr(), 0.0, 0.0, None)

    # -------------------------------------------------------------- conversion
    def numpy(self) -> np.ndarray:
        if self._device == "cpu":
            return self._host.copy()
        out = np.empty(self._shape, self._dtype)
        if out.nbytes:
            _C.call("lq_memcpy_d2h", out.ctypes.data, self.data_ptr(), out.nbytes, None)
        return out

    def item(self) -> Any:
        if self.numel() != 1:
            raise ValueError("item() needs a one-element tensor")
        return self.numpy().reshape(()).item()

    def tolist(self) -> Any:
        return self.numpy().tolist()

    def to(self, device: Any = None, dtype: Any = None) -> "Tensor":
        t = self
        if device is not None:
            dev = normalize_device(device)
            if dev != self._device:
                t = Tensor._from_numpy(self.numpy(), dev)
        if dtype is not None and np.dtype(dtype) != t._dtype:
            dt = np.dtype(dtype)
            if t._device != "cpu":
                if t._dtype not in FLOAT_TYPE_CODE or dt not in FLOAT_TYPE_CODE:
                    raise _C.LucidError("device dtype conversion is between float32, float16 and "
                                        f"bfloat16 only, not {t._dtype} -> {dt}")
                out = Tensor._empty(t._shape, dt, "gpu")
                _C.call("lq_cast", t.data_ptr(), FLOAT_TYPE_CODE[t._dtype], out.data_ptr(),
                        FLOAT_TYPE_CODE[dt], t.numel(), None)
                out.requires_grad = t.requires_grad
                return out
            t = Tensor._from_numpy(_host_astype(t._host, dt), "cpu")
        return t

    def cpu(self) -> "Tensor":
        return self.to("cpu")

    def gpu(self) -> "Tensor":
        return self.to("gpu")

    def record_stream(self, stream: Any) -> None:
        """Mark this device tensor's storage as used by work queued on ``stream`` (an
        ``lq_stream_create`` handle), so that when the storage is freed it is not handed out
        again before that work completes (``lq_record_stream``).  Device memory is freed on
        the null stream; work on a created stream is not ordered with it without this."""
        if self._device == "cpu":
            return
        if self._buf is None:
            self._materialize()
        _C.call("lq_record_stream", self._buf.ptr, stream)

    def detach(self) -> "Tensor":
        return self

    def contiguous(self) -> "Tensor":
        return self

    def clone(self) -> "Tensor":
        if self._device == "cpu":
            return Tensor._from_numpy(self._host, "cpu")
        t = Tensor._empty(self._shape, self._dtype, "gpu")
        if self.nbytes:
            _C.call("lq_memcpy_d2d", t._buf.ptr, self.data_ptr(), self.nbytes, None)
        return t

    def copy_(self, src: "Tensor") -> "Tensor":
        if tuple(src.shape) != self._shape:
            raise ValueError(f"copy_ shape mismatch {src.shape} vs {self._shape}")
        if src.dtype != self._dtype:
            raise ValueError(f"copy_ dtype mismatch {src.dtype} vs {self._dtype}")
        if self._device == "cpu":
            self._host[...] = src.numpy()
        elif self.nbytes:
            dst = self.data_ptr()
            if src.device == "cpu":
                arr = np.ascontiguousarray(src._host)
                _C.call("lq_memcpy_h2d", dst, arr.ctypes.data, arr.nbytes, None)
            else:
                _C.call("lq_memcpy_d2d", dst, src.data_ptr(), self.nbytes, None)
        self._qsrc = None
        return self

    def reshape(self, *shape: Any) -> "Tensor":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = tuple(int(s) for s in shape)
        n = self.numel()
        if -1 in shape:
            known = int(np.prod([s for s in shape if s != -1], dtype=np.int64))
            shape = tuple(n // known if s == -1 else s for s in shape)
        if int(np.prod(shape, dtype=np.int64)) != n:
            raise ValueError(f"cannot reshape {self._shape} to {shape}")
        t = Tensor()
        t._shape = shape
        t._dtype = self._dtype
        t._device = self._device
        t.requires_grad = self.requires_grad
        if self._device == "cpu":
            t._host = self._host.reshape(shape)
        else:
            if self._buf is None and self._qsrc is not None:
                q = self._qsrc
                t._qsrc = QuantSource(q.codes.reshape(shape), q.code_type, q.scale, q.zero_point,
                                      q.quant_min, q.quant_max)
            else:
                t._buf = self._buf
                t._offset = self._offset
                t._qsrc = self._qsrc
        return t

    def view(self, *shape: Any) -> "Tensor":
        return self.reshape(*shape)

    def flatten(self) -> "Tensor":
        return self.reshape(-1)

    def __len__(self) -> int:
        if not self._shape:
            raise TypeError("len() of a 0-d tensor")
        return self._shape[0]

    def __repr__(self) -> str:
        tag = ", code-backed" if self._qsrc is not None and self._buf is None else ""
        return f"Tensor(shape={self._shape}, dtype={self._dtype}, device='{self._device}'{tag})"

    def __deepcopy__(self, memo: dict) -> "Tensor":
        if self._device == "cpu":
            t = Tensor._from_numpy(self._host, "cpu")
        else:
            t = self.clone()
        t.requires_grad = self.requires_grad
        if type(self) is not Tensor:
            t.__class__ = type(self)
        return t

    def __reduce_ex__(self, protocol: int):
        return (_rebuild, (self.numpy(), self._device, type(self), self.requires_grad))


def _rebuild(arr: np.ndarray, device: str, cls: type, requires_grad: bool) -> Tensor:
    t = Tensor._from_numpy(arr, device)
    t.__class__ = cls
    t.requires_grad = requires_grad
    return t


# -------------------------------------------------------------------- factories


def tensor(data: Any, dtype: Any = None, device: Any = "cpu", requires_grad: bool = False) -> Tensor:
    if isinstance(data, Tensor):
        arr = data.numpy()
    else:
        arr = np.asarray(data)
    if dtype is not None:
        arr = _host_astype(arr, dtype)
    elif arr.dtype == np.float64:
        arr = arr.astype(np.float32)
    elif arr.dtype == np.int64 and not isinstance(data, np.ndarray):
        arr = arr.astype(np.int64)
    t = Tensor._from_numpy(arr, normalize_device(device))
    t.requires_grad = requires_grad
    return t


def from_numpy(arr: np.ndarray, device: Any = "cpu") -> Tensor:
    return Tensor._from_numpy(arr, normalize_device(device))


def empty(shape: Sequence[int] | int, dtype: Any = float32, device: Any = "cpu") -> Tensor:
    if isinstance(shape, int):
        shape = (shape,)
    return Tensor._empty(shape, np.dtype(dtype), normalize_device(device))


def full(shape: Sequence[int] | int, value: float, dtype: Any = float32, device: Any = "cpu") -> Tensor:
    if isinstance(shape, int):
        shape = (shape,)
    return tensor(np.full(shape, value, dtype=np.dtype(dtype)), device=device)


def zeros(shape: Sequence[int] | int, dtype: Any = float32, device: Any = "cpu") -> Tensor:
    return full(shape, 0, dtype, device)


def ones(shape: Sequence[int] | int, dtype: Any = float32, device: Any = "cpu") -> Tensor:
    return full(shape, 1, dtype, device)


def zeros_like(t: Tensor) -> Tensor:
    return zeros(t.shape, t.dtype, t.device)


def randn(*shape: Any, device: Any = "cpu", seed: int | None = None) -> Tensor:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    rng = np.random.default_rng(seed)
    return tensor(rng.standard_normal(shape, dtype=np.float32), device=device)
