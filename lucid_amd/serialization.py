"""SafeTensors checkpoints in Lucid's layout (lucid/serialization/__init__.py:833-990,
lucid/serialization/_safetensors.py).

The file is the standard SafeTensors container: an 8-byte little-endian header length, a JSON
header mapping each name to ``{"dtype", "shape", "data_offsets"}`` (plus optional string
``__metadata__``), space-padded so the data section starts 8-aligned, then the tensors' bytes
back to back in header order.  Lucid writes a zero-rank tensor (a quantized module's ``scale``
/ ``zero_point``) with shape ``[1]`` and lists its name, as a JSON list, under the metadata key
``__lucid_scalar_keys__``; loading restores those to zero rank.  So a quantized model's
``state_dict`` saved by Lucid loads here, and the other way round.

Loading validates the header as Lucid does (offsets forward, inside the data section, sized
for their shape and dtype, covering it without overlaps or gaps) and raises ``ValueError``
naming the file and tensor.  Unsigned integers widen as Lucid widens them (``U8`` to int16,
``U16`` to int32, ``U32`` / ``U64`` to int64, refusing uint64 values past int64); ``BF16``,
which numpy lacks, widens exactly to float32.
"""

from __future__ import annotations

import json
import math
import mmap
import os
import struct
from typing import Mapping

import numpy as np

from lucid_amd._tensor import Tensor, tensor

SCALAR_KEYS_KEY = "__lucid_scalar_keys__"
_METADATA_KEY = "__metadata__"

_CODES = {np.dtype(np.float64): "F64", np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
          np.dtype(np.int64): "I64", np.dtype(np.int32): "I32", np.dtype(np.int16): "I16",
          np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8", np.dtype(np.bool_): "BOOL",
          np.dtype(np.complex64): "C64"}
_NATIVE = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32,
           "I16": np.int16, "I8": np.int8, "BOOL": np.bool_, "C64": np.complex64}
_WIDEN = {"U8": (np.uint8, np.int16), "U16": (np.uint16, np.int32), "U32": (np.uint32, np.int64),
          "U64": (np.uint64, np.int64), "BF16": (np.uint16, np.float32)}


def _itemsize(code: str) -> int | None:
    if code in _NATIVE:
        return np.dtype(_NATIVE[code]).itemsize
    if code in _WIDEN:
        return np.dtype(_WIDEN[code][0]).itemsize
    return None


def _host_array(value: Tensor) -> np.ndarray:
    """The tensor's values on the host (a code-backed tensor materializes its floats)."""
    arr = value.numpy()
    return arr if arr.flags.c_contiguous else arr.copy(order="C")  # (ascontiguousarray would make 0-d 1-d)


def save_safetensors(state_dict: Mapping[str, object], path: str, *, metadata: dict[str, str] | None = None) -> None:
    """Write ``state_dict`` (name -> Tensor) as a SafeTensors file in Lucid's layout."""
    meta: dict[str, str] = {}
    for key, value in (metadata or {}).items():
        if not isinstance(value, str):
            raise TypeError(f"save_safetensors: metadata[{key!r}] must be a str, got {type(value).__name__}")
        if key == SCALAR_KEYS_KEY:
            raise ValueError(f"save_safetensors: metadata key {SCALAR_KEYS_KEY!r} is reserved")
        meta[key] = value
    header: dict[str, object] = {}
    blobs: list[bytes] = []
    scalars: list[str] = []
    offset = 0
    for name, value in state_dict.items():
        if not isinstance(value, Tensor):
            raise TypeError(f"save_safetensors: state_dict[{name!r}] is {type(value).__name__}, expected Tensor")
        arr = _host_array(value)
        code = _CODES.get(arr.dtype)
        if code is None:
            raise TypeError(f"save_safetensors: tensor {name!r} has dtype {arr.dtype}, which SafeTensors "
                            "cannot store")
        shape = [int(d) for d in arr.shape]
        if not shape:
            shape = [1]
            scalars.append(name)
        blob = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": code, "shape": shape, "data_offsets": [offset, offset + len(blob)]}
        blobs.append(blob)
        offset += len(blob)
    if scalars:
        meta[SCALAR_KEYS_KEY] = json.dumps(scalars, separators=(",", ":"))
    if meta:
        header[_METADATA_KEY] = meta
    encoded = json.dumps(header, separators=(",", ":")).encode("utf-8")
    encoded += b" " * (-len(encoded) % 8)
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(encoded)))
        fh.write(encoded)
        for blob in blobs:
            fh.write(blob)


def _decode_scalar_keys(text: str) -> frozenset[str]:
    """The names a scalar-keys value lists: a JSON list, or the legacy comma-joined form."""
    try:
        parsed = json.loads(text)
    except ValueError:
        parsed = None
    if isinstance(parsed, list) and all(isinstance(k, str) for k in parsed):
        return frozenset(parsed)
    return frozenset(k for k in text.split(",") if k)


class _File:
    def __init__(self, path: str | os.PathLike) -> None:
        self.path = os.fspath(path)
        with open(self.path, "rb") as fh:
            size = os.fstat(fh.fileno()).st_size
            prefix = fh.read(8)
            if len(prefix) != 8:
                raise self._error("too short to be SafeTensors")
            (hlen,) = struct.unpack("<Q", prefix)
            if hlen > size - 8:
                raise self._error(f"its header claims {hlen} bytes but the file holds only {size - 8} after the "
                                  "length prefix")
            try:
                header = json.loads(fh.read(hlen))
            except ValueError as exc:
                raise self._error("has no readable header") from exc
        if not isinstance(header, dict):
            raise self._error("its header is not a JSON object")
        self.base = 8 + hlen
        self.payload = size - self.base
        meta = header.pop(_METADATA_KEY, None) or {}
        if not isinstance(meta, dict) or not all(isinstance(k, str) and isinstance(v, str) for k, v in meta.items()):
            raise self._error(f"{_METADATA_KEY} must map strings to strings")
        self.metadata = meta
        self.scalar_keys = _decode_scalar_keys(meta.get(SCALAR_KEYS_KEY, ""))
        self.entries: dict[str, tuple[str, tuple[int, ...], int, int]] = {}
        for name, info in header.items():
            if not isinstance(info, dict):
                raise self._error("its record is not a JSON object", name)
            code, shape, offs = info.get("dtype"), info.get("shape"), info.get("data_offsets")
            if not isinstance(code, str):
                raise self._error("its record has no dtype string", name)
            if not isinstance(shape, list) or not all(isinstance(d, int) and not isinstance(d, bool) and d >= 0
                                                      for d in shape):
                raise self._error(f"its shape {shape!r} is not a list of non-negative ints", name)
            if not (isinstance(offs, list) and len(offs) == 2 and all(isinstance(o, int) for o in offs)):
                raise self._error(f"its data_offsets {offs!r} are not two ints", name)
            start, end = offs
            if start < 0 or end < start:
                raise self._error(f"its data_offsets [{start}, {end}] are not a forward range", name)
            if end > self.payload:
                raise self._error(f"its bytes [{start}, {end}) run past the {self.payload}-byte data section "
                                  "(the file is truncated or the header is wrong)", name)
            width = _itemsize(code)
            if width is None:
                raise self._error(f"stored as {code}, which this backend cannot represent", name)
            need = math.prod(shape) * width
            if end - start != need:
                raise self._error(f"shape {shape} of {code} needs {need} bytes but its data_offsets span "
                                  f"{end - start}", name)
            self.entries[name] = (code, tuple(shape), start, end)
        cursor, previous = 0, None
        for name, (_, _, start, end) in sorted(self.entries.items(), key=lambda kv: (kv[1][2], kv[1][3])):
            if start < cursor:
                raise self._error(f"its bytes [{start}, {end}) overlap {previous!r}", name)
            if start > cursor:
                raise self._error(f"{start - cursor} bytes before it belong to no tensor", name)
            cursor, previous = end, name
        if cursor != self.payload:
            raise self._error(f"{self.payload - cursor} trailing bytes follow the last tensor")

    def _error(self, what: str, name: str | None = None) -> ValueError:
        where = f" (tensor {name!r})" if name is not None else ""
        return ValueError(f"{self.path}: not a valid SafeTensors file: {what}{where}")

    def decode(self, name: str, raw: bytes) -> np.ndarray:
        code, shape, _, _ = self.entries[name]
        if code in _NATIVE:
            arr = np.frombuffer(raw, dtype=np.dtype(_NATIVE[code]).newbyteorder("<")).astype(_NATIVE[code])
        else:
            stored, target = _WIDEN[code]
            vals = np.frombuffer(raw, dtype=np.dtype(stored).newbyteorder("<"))
            if code == "BF16":
                arr = (vals.astype(np.uint32) << 16).view(np.float32)
            else:
                if code == "U64" and vals.size and int(vals.max()) > 2 ** 63 - 1:
                    raise self._error("holds uint64 values past int64's range", name)
                arr = vals.astype(target)
        arr = arr.reshape(shape)
        if name in self.scalar_keys and shape == (1,):
            arr = arr.reshape(())
        return arr


def load_safetensors(path: str | os.PathLike, *, device: str = "cpu") -> dict[str, Tensor]:
    """Read every tensor of a SafeTensors file (Lucid's layout) onto ``device``."""
    f = _File(path)
    out: dict[str, Tensor] = {}
    if not f.entries:
        return out
    with open(f.path, "rb") as fh, mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as data:
        for name, (_, _, start, end) in f.entries.items():
            arr = f.decode(name, bytes(data[f.base + start:f.base + end]))
            out[name] = tensor(arr, device=device)
    return out


class safe_open:
    """Lazy reader (``keys()``, ``get_tensor(name)``, ``metadata()``), a context manager like
    Lucid's (lucid/serialization/__init__.py:984-): the header is validated on open, each
    tensor read when asked for."""

    def __init__(self, filename: str | os.PathLike, framework: str = "lucid", device: str = "cpu") -> None:
        self._f = _File(filename)
        self._device = device

    def __enter__(self) -> "safe_open":
        return self

    def __exit__(self, *exc) -> None:
        return None

    def keys(self) -> list[str]:
        return list(self._f.entries)

    def metadata(self) -> dict[str, str]:
        return dict(self._f.metadata)

    def get_tensor(self, name: str) -> Tensor:
        _, _, start, end = self._f.entries[name]
        with open(self._f.path, "rb") as fh:
            fh.seek(self._f.base + start)
            raw = fh.read(end - start)
        return tensor(self._f.decode(name, raw), device=self._device)
