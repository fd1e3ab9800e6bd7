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

``save`` / ``load`` write and read Lucid's own checkpoint format
(lucid/serialization/__init__.py:105-456): a pickle stream of the container
``{"_lucid_format": 2, "obj": obj[, "_state_dict_metadata": ...]}`` in which every tensor is a
persistent id, ``("tensor_v3", tid, shape, stride, offset, dtype name, device, is_param,
requires_grad, storage id, bytes)`` -- shape / stride / offset in elements, the storage's raw
bytes on its first record only -- or ``("tensor_ref", tid)`` for a tensor written before.
Loading accepts the older records (``("tensor_v3", shape, dtype, device, bytes)`` and
``("tensor", shape, dtype, device, bytes, numpy dtype)``) and rebuilds views of shared
storages.  By default (``weights_only=True``) only the globals Lucid's restricted unpickler
allows are resolved (builtins containers and scalars, ``collections`` dicts, numpy arrays /
dtypes / scalars, Lucid's dtype constants); anything else raises ``pickle.UnpicklingError``.
"""

from __future__ import annotations

import io
import json
import math
import mmap
import os
import pickle
import struct
import warnings
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


# ------------------------------------------------------------ Lucid's pickle checkpoints

# Lucid's dtype names (lucid/_dtype.py:85-100) and their numpy storage; bfloat16, which numpy
# lacks, is read as the upper halves of float32 words.
_LUCID_DTYPES = {"float16": np.float16, "float32": np.float32, "float64": np.float64, "int8": np.int8,
                 "int16": np.int16, "int32": np.int32, "int64": np.int64, "bool": np.bool_,
                 "bool_": np.bool_, "complex64": np.complex64, "complex128": np.complex128}
_NUMPY_TO_LUCID = {np.dtype(v): k for k, v in _LUCID_DTYPES.items() if k != "bool_"}

# Globals the restricted loader resolves (lucid/serialization/__init__.py:33-80).
_SAFE_GLOBALS = {
    ("builtins", n) for n in ("dict", "list", "tuple", "int", "float", "complex", "str", "bool", "bytes",
                              "bytearray", "set", "slice", "NoneType")
} | {("collections", n) for n in ("OrderedDict", "Counter", "defaultdict")} | {
    ("numpy", "ndarray"), ("numpy", "dtype"), ("numpy.core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"), ("numpy._core.multiarray", "_reconstruct"),
    ("numpy._core.multiarray", "scalar")}


def _lucid_device(t: Tensor) -> str:
    # Lucid's accelerator is named "metal"; a device tensor saved here loads onto Lucid's GPU
    return "metal" if t.device == "gpu" else "cpu"


class _Pickler(pickle.Pickler):
    """Each tensor becomes a dense storage of its own (no sharing is claimed)."""

    def __init__(self, file, protocol: int) -> None:
        super().__init__(file, protocol=protocol)
        self._emitted: dict[int, int] = {}
        self._alive: list[Tensor] = []

    def persistent_id(self, obj: object):
        if not isinstance(obj, Tensor):
            return None
        tid = self._emitted.get(id(obj))
        if tid is not None:
            return ("tensor_ref", tid)
        tid = len(self._emitted)
        self._emitted[id(obj)] = tid
        self._alive.append(obj)  # ids stay unique while the dump runs
        arr = _host_array(obj)
        name = _NUMPY_TO_LUCID.get(arr.dtype)
        if name is None:
            raise TypeError(f"save: no Lucid dtype for {arr.dtype}")
        shape = [int(d) for d in arr.shape]
        stride, acc = [], 1
        for d in reversed(shape):
            stride.append(acc)
            acc *= max(d, 1)
        stride.reverse()
        from lucid_amd.nn.module import Parameter

        return ("tensor_v3", tid, shape, stride, 0, name, _lucid_device(obj), isinstance(obj, Parameter),
                bool(obj.requires_grad), tid, arr.tobytes())


def save(obj: object, f, pickle_module: object = pickle, pickle_protocol: int = 4) -> None:
    """Write ``obj`` (a state_dict, or any picklable structure holding tensors) as a Lucid
    checkpoint (lucid/serialization/__init__.py:287-360)."""
    if pickle_module not in (None, pickle):
        raise NotImplementedError("save supports only the standard pickle module")
    container: dict[str, object] = {"_lucid_format": 2, "obj": obj}
    meta = getattr(obj, "_metadata", None)
    if meta is not None:
        container["_state_dict_metadata"] = meta
    buf = io.BytesIO()
    _Pickler(buf, pickle_protocol).dump(container)
    if isinstance(f, (str, bytes, os.PathLike)):
        with open(os.fspath(f), "wb") as fp:
            fp.write(buf.getvalue())
    else:
        f.write(buf.getvalue())


def _target(device_str: str, map_location: object) -> str:
    from lucid_amd._tensor import normalize_device

    if isinstance(map_location, dict):
        return normalize_device(map_location.get(device_str, device_str))
    if isinstance(map_location, str):
        return normalize_device(map_location)
    return normalize_device(device_str)


def _storage_array(raw: object, name: str, where: str) -> np.ndarray:
    if name == "bfloat16":
        if not isinstance(raw, (bytes, bytearray)) or len(raw) % 2:
            raise pickle.UnpicklingError(f"{where}: bfloat16 storage with an odd byte count")
        return (np.frombuffer(bytes(raw), np.uint16).astype(np.uint32) << 16).view(np.float32)
    if name not in _LUCID_DTYPES:
        raise pickle.UnpicklingError(f"{where}: unknown dtype {name!r}")
    dt = np.dtype(_LUCID_DTYPES[name])
    if not isinstance(raw, (bytes, bytearray)) or len(raw) % dt.itemsize:
        raise pickle.UnpicklingError(f"{where}: storage has no bytes, or a byte count that is not a multiple of "
                                     f"{name}'s {dt.itemsize}")
    return np.frombuffer(bytes(raw), dt)


def _view(storage: np.ndarray, shape, stride, offset, where: str) -> np.ndarray:
    shape = [int(d) for d in shape]
    stride = [int(s) for s in stride]
    offset = int(offset)
    if len(shape) != len(stride) or any(d < 0 for d in shape) or any(s < 0 for s in stride) or offset < 0:
        raise pickle.UnpicklingError(f"{where}: bad view geometry")
    if math.prod(shape) == 0:
        return np.zeros(shape, storage.dtype)
    last = offset + sum((d - 1) * s for d, s in zip(shape, stride))
    if last >= storage.size:
        raise pickle.UnpicklingError(f"{where}: view reaches element {last} of a storage of {storage.size}")
    it = storage.itemsize
    return np.lib.stride_tricks.as_strided(storage[offset:], shape=shape, strides=[s * it for s in stride]).copy()


class _Unpickler(pickle.Unpickler):
    def __init__(self, file, map_location: object, safe: bool, **kw) -> None:
        super().__init__(file, **kw)
        self._map = map_location
        self._safe = safe
        self._storages: dict[int, np.ndarray] = {}
        self._tensors: dict[int, Tensor] = {}

    def find_class(self, module: str, name: str):
        if module == "lucid._dtype" and name in _LUCID_DTYPES:
            return np.dtype(_LUCID_DTYPES[name])
        if self._safe and (module, name) not in _SAFE_GLOBALS:
            raise pickle.UnpicklingError(f"weights_only=True: refusing to deserialize '{module}.{name}'. "
                                         "Pass weights_only=False to allow arbitrary objects "
                                         "(potential security risk).")
        return super().find_class(module, name)

    def _make(self, arr: np.ndarray, device_str: str, is_param: bool = False, requires_grad: bool = False) -> Tensor:
        t = Tensor._from_numpy(arr, _target(device_str, self._map))
        if is_param:
            from lucid_amd.nn.module import Parameter

            t = Parameter(t, bool(requires_grad))
        t.requires_grad = bool(requires_grad)
        if callable(self._map) and not isinstance(self._map, (str, dict)):
            t = self._map(t, device_str)
        return t

    def persistent_load(self, pid: object):
        if isinstance(pid, tuple) and pid:
            tag = pid[0]
            if tag == "tensor_ref" and len(pid) == 2:
                tid = int(pid[1])
                if tid not in self._tensors:
                    raise pickle.UnpicklingError(f"reference to tensor record {tid} before it")
                return self._tensors[tid]
            if tag == "tensor_v3" and len(pid) == 11:
                _, tid, shape, stride, offset, name, dev, is_param, rg, sid, raw = pid
                where = f"tensor record {tid}"
                base = self._storages.get(int(sid))
                if base is None:
                    base = _storage_array(raw, name, where)
                    self._storages[int(sid)] = base
                t = self._make(_view(base, shape, stride, offset, where), dev, is_param, rg)
                self._tensors[int(tid)] = t
                return t
            if tag == "tensor_v3" and len(pid) == 5:
                _, shape, name, dev, raw = pid
                arr = _storage_array(raw, name, "tensor record")
                return self._make(arr.reshape([int(d) for d in shape]), dev)
            if tag == "tensor" and len(pid) == 6:
                _, shape, name, dev, raw, _np = pid
                arr = _storage_array(raw, name, "tensor record")
                return self._make(arr.reshape([int(d) for d in shape]), dev)
        raise pickle.UnpicklingError(f"Unknown persistent id: {pid}")


def _no_frozenset(obj: object, seen: set[int]) -> None:
    if id(obj) in seen:
        return
    if isinstance(obj, frozenset):
        raise pickle.UnpicklingError("weights_only=True: refusing to deserialize 'builtins.frozenset'.")
    if isinstance(obj, dict):
        seen.add(id(obj))
        for k, v in obj.items():
            _no_frozenset(k, seen)
            _no_frozenset(v, seen)
    elif isinstance(obj, (list, tuple, set)):
        seen.add(id(obj))
        for v in obj:
            _no_frozenset(v, seen)


def load(f, map_location: object = None, pickle_module: object = None, *, weights_only: bool | None = True,
         mmap: bool | None = None, **pickle_load_args):
    """Read a checkpoint written by ``save`` (or by Lucid's ``lucid.save``), or a
    ``.safetensors`` file (lucid/serialization/__init__.py:361-456).

    ``map_location``: None (each tensor where it was saved: "metal" / "gpu" on the GPU), a
    device name for every tensor, a dict from saved device name to target, or a callable
    ``fn(tensor, saved_device) -> tensor``."""
    if pickle_module not in (None, pickle):
        raise NotImplementedError("load supports only the standard pickle module")
    if mmap is True:
        raise NotImplementedError("load does not support mmap=True")
    safe = True if weights_only is None else bool(weights_only)
    if safe and pickle_load_args:
        raise RuntimeError("Cannot use ``pickle_load_args`` with ``weights_only=True``")
    if map_location is not None and not (isinstance(map_location, (str, dict)) or callable(map_location)):
        raise TypeError("map_location must be a device name, a dict of them or a callable, got "
                        f"{type(map_location).__name__}")
    if isinstance(f, (str, bytes, os.PathLike)):
        path = os.fspath(f)
        path = path.decode() if isinstance(path, bytes) else path
        if path.endswith(".safetensors"):
            out = load_safetensors(path)
            if map_location is None:
                return out
            return {k: Tensor._from_numpy(v.numpy(), _target(v.device, map_location)) for k, v in out.items()}
        with open(path, "rb") as fp:
            data = fp.read()
    else:
        data = f.read()
    if not safe:
        warnings.warn("load() with weights_only=False allows arbitrary object deserialization which may "
                      "execute untrusted code.", UserWarning, stacklevel=2)
    container = _Unpickler(io.BytesIO(data), map_location, safe, **pickle_load_args).load()
    if safe:
        _no_frozenset(container, set())
    if not isinstance(container, dict) or container.get("_lucid_format") not in (1, 2):
        raise RuntimeError("File is not a valid Lucid checkpoint")
    obj = container["obj"]
    meta = container.get("_state_dict_metadata")
    if meta is not None and isinstance(obj, dict):
        try:
            obj._metadata = meta
        except AttributeError:
            from collections import OrderedDict

            obj = OrderedDict(obj)
            obj._metadata = meta
    return obj


# ------------------------------------------------------------------ sharded checkpoints


def _directory_of(path: object, caller: str) -> str:
    """The directory a sharded checkpoint lives in: a str, bytes or os.PathLike path, and
    nothing else (anything at all can be str()-ed into a path name by mistake)."""
    try:
        return os.fsdecode(os.fspath(path))
    except TypeError:
        raise TypeError(f"{caller}() expects a directory path as str, bytes or os.PathLike, got "
                        f"{type(path).__name__}") from None


def _tensors_in(v: object, out: dict[int, Tensor], seen: set[int]) -> None:
    if id(v) in seen:
        return
    seen.add(id(v))
    if isinstance(v, Tensor):
        out[id(v)] = v
    elif isinstance(v, dict):
        for k, x in v.items():
            _tensors_in(k, out, seen)
            _tensors_in(x, out, seen)
    elif isinstance(v, (list, tuple, set, frozenset)):
        for x in v:
            _tensors_in(x, out, seen)


def _shard_groups(obj: dict) -> list[tuple[list[str], int]]:
    """Keys grouped by the tensors they reach (a tensor reached from two keys -- a tied weight --
    joins them), each group with the bytes of its distinct tensors, in first-key order
    (lucid/serialization/_storage_plan.py:455-482; tensors here share memory only by identity)."""
    parent: dict[str, str] = {}

    def find(k: str) -> str:
        while parent[k] != k:
            parent[k] = parent[parent[k]]
            k = parent[k]
        return k

    owner: dict[int, str] = {}
    reach: dict[str, dict[int, Tensor]] = {}
    for k, v in obj.items():
        parent[k] = k
        reach[k] = {}
        _tensors_in(v, reach[k], set())
        for tid in reach[k]:
            if tid in owner:
                parent[find(k)] = find(owner[tid])
            else:
                owner[tid] = k
    groups: dict[str, list[str]] = {}
    for k in obj:
        groups.setdefault(find(k), []).append(k)
    out = []
    for keys in groups.values():
        distinct: dict[int, Tensor] = {}
        for k in keys:
            distinct.update(reach[k])
        out.append((keys, sum(t.numel() * np.dtype(t.dtype).itemsize for t in distinct.values())))
    return out


_INDEX = "index.json"
_SHARDED_TAG = "_lucid_sharded"


def _shard_file(i: int, n: int) -> str:
    return f"shard-{i:05d}-of-{n:05d}.lucid"


def _plan_shards(obj: dict, cap_bytes: int) -> list[list[str]]:
    """Keys per shard: key groups (keys reaching a shared tensor stay together) in first-key
    order, a new shard opened whenever the next group would push a non-empty shard past the
    cap (a group over the cap alone gets its own shard); at least one shard."""
    plan: list[list[str]] = [[]]
    used = 0
    for keys, nbytes in _shard_groups(obj):
        if plan[-1] and used + nbytes > cap_bytes:
            plan.append([])
            used = 0
        plan[-1].extend(keys)
        used += nbytes
    return plan


def _write_index(directory: str, doc: dict) -> None:
    with open(os.path.join(directory, _INDEX), "w", encoding="utf-8") as fp:
        json.dump(doc, fp, indent=2)


def save_sharded(obj: object, path, *, shard_size_mb: float = 1024.0, pickle_protocol: int = 4) -> None:
    """A checkpoint directory of ``shard-XXXXX-of-YYYYY.lucid`` files, each a ``save`` of part of
    a state dict, plus an ``index.json`` naming each shard's keys -- Lucid's sharded layout
    (lucid/serialization/__init__.py:646-744).  Keys are packed first-fit up to
    ``shard_size_mb``; keys that share a tensor stay in one shard.  A non-dict object is one
    shard whose index entry lists no keys.  The index also carries the dict's key order when
    packing moved a key, and its ``_metadata`` when that is JSON-serialisable."""
    directory = _directory_of(path, "save_sharded")
    os.makedirs(directory, exist_ok=True)
    if not isinstance(obj, dict):
        name = _shard_file(0, 1)
        save(obj, os.path.join(directory, name), pickle_protocol=pickle_protocol)
        _write_index(directory, {_SHARDED_TAG: 1, "shards": [{"file": name, "keys": None}]})
        return
    plan = _plan_shards(obj, int(shard_size_mb * 1024 * 1024))
    doc: dict[str, object] = {_SHARDED_TAG: 1, "shards": []}
    for i, keys in enumerate(plan):
        name = _shard_file(i, len(plan))
        save({k: obj[k] for k in keys}, os.path.join(directory, name), pickle_protocol=pickle_protocol)
        doc["shards"].append({"file": name, "keys": list(keys)})
    order = list(obj)
    if sum(plan, []) != order:
        doc["key_order"] = order
    meta = getattr(obj, "_metadata", None)
    if meta is not None:
        try:
            doc["_state_dict_metadata"] = json.loads(json.dumps(meta))
        except (TypeError, ValueError):
            pass  # metadata that JSON cannot carry is left out
    _write_index(directory, doc)


def _read_index(directory: str) -> dict:
    """A sharded checkpoint's index document, validated (tag, plain shard file names)."""
    index_path = os.path.join(directory, _INDEX)
    with open(index_path, encoding="utf-8") as fp:
        doc = json.load(fp)
    if not isinstance(doc, dict) or doc.get(_SHARDED_TAG) != 1:
        raise RuntimeError(f"{index_path!r} is not a valid Lucid sharded checkpoint index")
    entries = doc["shards"]
    for entry in entries:  # shard files stay inside the directory
        name = str(entry["file"])
        if name in ("", ".", "..") or os.path.basename(name) != name:
            raise RuntimeError(f"{index_path!r}: shard file {name!r} is not a plain file name")
    return doc


def load_sharded(path, *, map_location: object = None, weights_only: bool = True) -> object:
    """Read a directory written by ``save_sharded`` (or by Lucid) back into one ordered state
    dict -- shards in index order, the recorded key order and metadata restored -- or the
    single object of a key-less one-shard index (lucid/serialization/__init__.py:746-830)."""
    from collections import OrderedDict

    directory = _directory_of(path, "load_sharded")
    doc = _read_index(directory)
    entries = doc["shards"]

    def read(entry: dict) -> object:
        return load(os.path.join(directory, str(entry["file"])), map_location=map_location,
                    weights_only=weights_only)

    if len(entries) == 1 and entries[0].get("keys") is None:
        return read(entries[0])
    merged: OrderedDict = OrderedDict()
    for part in map(read, entries):
        if isinstance(part, dict):
            merged.update(part)
    order = doc.get("key_order")
    if isinstance(order, list) and set(order) == set(merged):
        merged = OrderedDict((k, merged[k]) for k in order)
    meta = doc.get("_state_dict_metadata")
    if isinstance(meta, dict):
        merged._metadata = meta
    return merged
