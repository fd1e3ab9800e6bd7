"""SafeTensors checkpoints in Lucid's layout (lucid_amd/serialization.py).

Pinned by the format itself: the third-party ``safetensors`` reader and writer (the published
implementation of the container) read what this module writes and write what it reads; the
Lucid-specific part (zero-rank tensors stored as shape [1] and listed, as a JSON list, under
``__lucid_scalar_keys__``, lucid/serialization/__init__.py:883-905) is checked byte for byte.
"""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from lucid_amd import serialization as S
from lucid_amd._tensor import tensor


def _sd():
    rng = np.random.default_rng(0)
    return {
        "weight_int8": tensor(rng.integers(-128, 128, (4, 6)).astype(np.int8)),
        "weight_scale": tensor(rng.uniform(0.01, 0.1, 4).astype(np.float32)),
        "bias": tensor(rng.standard_normal(4).astype(np.float32)),
        "scale": tensor(np.float32(0.037)),
        "zero_point": tensor(np.float32(128.0)),
        "num_batches_tracked": tensor(np.array(7, np.int64)),
        "mask": tensor(np.array([True, False, True])),
        "half": tensor(np.arange(5, dtype=np.float16)),
    }


def test_round_trip_and_layout(tmp_path):
    sd = _sd()
    path = tmp_path / "m.safetensors"
    S.save_safetensors(sd, str(path), metadata={"format": "pt"})
    raw = path.read_bytes()
    (hlen,) = struct.unpack("<Q", raw[:8])
    assert (8 + hlen) % 8 == 0
    header = json.loads(raw[8:8 + hlen])
    assert header["scale"] == {"dtype": "F32", "shape": [1], "data_offsets": header["scale"]["data_offsets"]}
    assert json.loads(header["__metadata__"]["__lucid_scalar_keys__"]) == ["scale", "zero_point",
                                                                           "num_batches_tracked"]
    assert header["__metadata__"]["format"] == "pt"
    back = S.load_safetensors(str(path))
    assert list(back) == list(sd)
    for k, v in sd.items():
        got = back[k].numpy()
        assert got.dtype == v.numpy().dtype and got.shape == v.numpy().shape, k
        np.testing.assert_array_equal(got, v.numpy())
    with S.safe_open(str(path)) as f:
        assert f.keys() == list(sd) and f.metadata()["format"] == "pt"
        assert f.get_tensor("zero_point").numpy().shape == ()


def test_interop_with_the_safetensors_library(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    sd = _sd()
    ours = tmp_path / "ours.safetensors"
    S.save_safetensors(sd, str(ours))
    theirs_read = st.load_file(str(ours))
    for k, v in sd.items():
        want = v.numpy().reshape(-1) if v.numpy().ndim == 0 else v.numpy()
        np.testing.assert_array_equal(theirs_read[k], want)
    # a file written by the library; unsigned bytes widen to int16 as Lucid widens them
    theirs = tmp_path / "theirs.safetensors"
    st.save_file({"a": np.arange(6, dtype=np.float32).reshape(2, 3), "u": np.array([0, 200, 255], np.uint8),
                  "i": np.array([-3, 4], np.int64)}, str(theirs))
    back = S.load_safetensors(str(theirs))
    np.testing.assert_array_equal(back["a"].numpy(), np.arange(6, dtype=np.float32).reshape(2, 3))
    assert back["u"].numpy().dtype == np.int16 and back["u"].numpy().tolist() == [0, 200, 255]
    assert back["i"].numpy().tolist() == [-3, 4]


def _write(path, header, payload):
    enc = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(enc)) + enc + payload)


@pytest.mark.parametrize("header,payload,msg", [
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4, "run past"),
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4, "needs 8 bytes"),
    ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
      "b": {"dtype": "F32", "shape": [1], "data_offsets": [2, 6]}}, b"\0" * 6, "overlap"),
    ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8, "belong to no tensor"),
    ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 8, "trailing bytes"),
    ({"a": {"dtype": "F8_E4M3", "shape": [1], "data_offsets": [0, 1]}}, b"\0", "cannot represent"),
])
def test_malformed_files_are_refused(tmp_path, header, payload, msg):
    p = tmp_path / "bad.safetensors"
    _write(p, header, payload)
    with pytest.raises(ValueError, match=msg):
        S.load_safetensors(str(p))


def test_bf16_widens_exactly(tmp_path):
    vals = np.array([1.0, -2.5, 3.140625, 1e-30], np.float32)
    bf = (vals.view(np.uint32) >> 16).astype(np.uint16)   # exact: these fit bfloat16 ... or truncate
    p = tmp_path / "bf.safetensors"
    _write(p, {"w": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}, bf.tobytes())
    got = S.load_safetensors(str(p))["w"].numpy()
    np.testing.assert_array_equal(got, (bf.astype(np.uint32) << 16).view(np.float32))


@pytest.mark.gpu
def test_quantized_model_checkpoint_round_trip(gpu, tmp_path):
    # a converted static conv stack saved and loaded into a freshly converted copy: the same
    # codes out
    from tests.test_gpu_modules import _conv_pipeline

    rng, _, q = _conv_pipeline(gpu)
    _, _, fresh = _conv_pipeline(gpu, seed=99)
    path = tmp_path / "q.safetensors"
    S.save_safetensors(q.state_dict(), str(path))
    fresh.load_state_dict(S.load_safetensors(str(path), device="gpu"))
    x = gpu.tensor(rng.standard_normal((2, 3, 16, 16)).astype(np.float32), device="gpu")
    np.testing.assert_array_equal(fresh(x).quant_source.codes.numpy(), q(x).quant_source.codes.numpy())


# ------------------------------------------------ Lucid's pickle checkpoints (save / load)
#
# Pinned against the record layout of lucid/serialization/__init__.py:113-152 (what Lucid's
# pickler writes) and :186-227 (what its loader accepts): the files are read back here by a
# bare pickle.Unpickler that only records the persistent ids, and files in Lucid's layout
# with shared storages and strided views -- which this module's writer never emits -- are
# built by hand and loaded.


class _Recorder(__import__("pickle").Unpickler):
    def __init__(self, f):
        super().__init__(f)
        self.pids = []

    def persistent_load(self, pid):
        self.pids.append(pid)
        return ("PID", len(self.pids) - 1)


def test_lucid_save_records_and_round_trip(tmp_path):
    import io
    import pickle
    from collections import OrderedDict

    import lucid_amd

    sd = OrderedDict(_sd())
    sd["again"] = sd["bias"]                      # the same tensor twice -> tensor_ref
    sd["extra"] = {"step": 3, "names": ["a", "b"], "lr": 0.5}
    path = tmp_path / "m.lucid"
    lucid_amd.save(sd, str(path))
    rec = _Recorder(io.BytesIO(path.read_bytes()))
    container = rec.load()
    assert container["_lucid_format"] == 2 and list(container["obj"]) == list(sd)
    v3 = [p for p in rec.pids if p[0] == "tensor_v3"]
    refs = [p for p in rec.pids if p[0] == "tensor_ref"]
    assert len(v3) == len(_sd()) and refs == [("tensor_ref", 2)]
    for tid, (name, t) in enumerate(list(_sd().items())):
        p = v3[tid]
        arr = t.numpy()
        assert len(p) == 11 and p[1] == tid and p[9] == tid
        assert p[2] == list(arr.shape) and p[4] == 0 and p[6] == "cpu" and p[7] is False and p[8] is False
        assert p[3] == [int(s) // arr.itemsize for s in arr.strides] or arr.ndim == 0
        assert p[5] == {"bool": "bool"}.get(arr.dtype.name, arr.dtype.name)
        assert p[10] == arr.tobytes()
    back = lucid_amd.load(str(path))
    assert list(back) == list(sd) and back["extra"] == sd["extra"]
    assert back["again"] is back["bias"]
    for k, t in _sd().items():
        got = back[k].numpy()
        assert got.dtype == t.numpy().dtype and got.shape == t.numpy().shape
        np.testing.assert_array_equal(got, t.numpy())
    # state_dict metadata round-trips (format v2)
    sd2 = OrderedDict(w=tensor(np.ones(2, np.float32)))
    sd2._metadata = {"": {"version": 1}}
    buf = io.BytesIO()
    S.save(sd2, buf)
    assert S.load(io.BytesIO(buf.getvalue()))._metadata == {"": {"version": 1}}
    assert pickle.loads  # the module is the standard one


def _lucid_file(obj, records):
    """A checkpoint in Lucid's layout: ``records`` maps a placeholder string inside ``obj`` to the
    persistent id Lucid's pickler would emit for it."""
    import io
    import pickle

    class P(pickle.Pickler):
        def persistent_id(self, o):
            return records.get(o) if isinstance(o, str) else None

    buf = io.BytesIO()
    P(buf, protocol=4).dump({"_lucid_format": 2, "obj": obj})
    return buf.getvalue()


def _ph(rec):
    """Placeholders "@K" for the records (dict keys stay plain names)."""
    return {k.lower(): "@" + k for k in rec}, {"@" + k: v for k, v in rec.items()}


def test_lucid_load_shared_storage_views_and_old_records():
    import io

    base = np.arange(24, dtype=np.float32)
    raw = base.tobytes()
    rec = {
        "A": ("tensor_v3", 0, [4, 6], [6, 1], 0, "float32", "cpu", True, True, 7, raw),
        "AT": ("tensor_v3", 1, [6, 4], [1, 6], 0, "float32", "cpu", False, False, 7, None),   # transpose view
        "ROW": ("tensor_v3", 2, [3], [2], 13, "float32", "cpu", False, False, 7, None),      # strided slice
        "REF": ("tensor_ref", 1),
        "OLD5": ("tensor_v3", [2, 2], "int16", "cpu", np.array([1, -2, 3, -4], np.int16).tobytes()),
        "OLD6": ("tensor", [3], "int8", "cpu", np.array([5, -6, 7], np.int8).tobytes(), "int8"),
        "BF": ("tensor_v3", 3, [2], [1], 0, "bfloat16", "cpu", False, False, 8,
               np.array([0x3FC0, 0xC040], np.uint16).tobytes()),
    }
    out = S.load(io.BytesIO(_lucid_file(*_ph(rec))))
    out = {k.upper(): v for k, v in out.items()}
    from lucid_amd.nn.module import Parameter

    A = base.reshape(4, 6)
    assert isinstance(out["A"], Parameter) and out["A"].requires_grad
    np.testing.assert_array_equal(out["A"].numpy(), A)
    np.testing.assert_array_equal(out["AT"].numpy(), A.T)
    np.testing.assert_array_equal(out["ROW"].numpy(), base[13:18:2])
    assert out["REF"] is out["AT"]
    np.testing.assert_array_equal(out["OLD5"].numpy(), [[1, -2], [3, -4]])
    np.testing.assert_array_equal(out["OLD6"].numpy(), [5, -6, 7])
    np.testing.assert_array_equal(out["BF"].numpy(), np.array([1.5, -3.0], np.float32))


def test_lucid_load_refuses_unsafe_and_damaged_files():
    import io
    import os
    import pickle

    class Evil:
        def __reduce__(self):
            return (os.getcwd, ())

    buf = io.BytesIO()
    pickle.dump({"_lucid_format": 2, "obj": Evil()}, buf, protocol=4)
    with pytest.raises(pickle.UnpicklingError, match="refusing"):
        S.load(io.BytesIO(buf.getvalue()))
    with pytest.warns(UserWarning):
        assert S.load(io.BytesIO(buf.getvalue()), weights_only=False) == os.getcwd()
    buf = io.BytesIO()
    pickle.dump({"_lucid_format": 2, "obj": frozenset({1})}, buf, protocol=4)
    with pytest.raises(pickle.UnpicklingError, match="frozenset"):
        S.load(io.BytesIO(buf.getvalue()))
    bad = {"X": ("tensor_v3", 0, [2], [1], 0, "float32", "cpu", False, False, 0, b"\0" * 7)}
    with pytest.raises(pickle.UnpicklingError, match="multiple"):
        S.load(io.BytesIO(_lucid_file(*_ph(bad))))
    far = {"X": ("tensor_v3", 0, [3], [4], 0, "float32", "cpu", False, False, 0, b"\0" * 16)}
    with pytest.raises(pickle.UnpicklingError, match="reaches"):
        S.load(io.BytesIO(_lucid_file(*_ph(far))))
    buf = io.BytesIO()
    pickle.dump({"not": "lucid"}, buf, protocol=4)
    with pytest.raises(RuntimeError, match="not a valid Lucid checkpoint"):
        S.load(io.BytesIO(buf.getvalue()))
    with pytest.raises(RuntimeError, match="pickle_load_args"):
        S.load(io.BytesIO(buf.getvalue()), encoding="latin1")


def test_lucid_load_dispatches_safetensors_and_maps_devices(tmp_path):
    path = tmp_path / "m.safetensors"
    S.save_safetensors(_sd(), str(path))
    out = S.load(str(path))
    np.testing.assert_array_equal(out["weight_int8"].numpy(), _sd()["weight_int8"].numpy())
    import io

    rec = {"G": ("tensor_v3", 0, [2], [1], 0, "int32", "metal", False, False, 0, np.array([1, 2], np.int32).tobytes())}
    out = S.load(io.BytesIO(_lucid_file(*_ph(rec))), map_location={"metal": "cpu"})
    assert out["g"].device == "cpu"
    np.testing.assert_array_equal(out["g"].numpy(), [1, 2])
    out = S.load(io.BytesIO(_lucid_file(*_ph(rec))), map_location="cpu")
    assert out["g"].device == "cpu"
    seen = []
    rec_c = {"G": rec["G"][:6] + ("cpu",) + rec["G"][7:]}
    out = S.load(io.BytesIO(_lucid_file(*_ph(rec_c))), map_location=lambda t, d: seen.append(d) or t)
    assert seen == ["cpu"] and out["g"].device == "cpu"


@pytest.mark.gpu
def test_lucid_checkpoint_of_device_tensors(gpu, tmp_path):
    """Device tensors are recorded as Lucid's accelerator ("metal") and load back onto the GPU."""
    import io

    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd

    m = nnqd.Linear.from_float(nn.Linear(16, 8).to("gpu")) if hasattr(nnqd, "Linear") else None
    sd = m.state_dict() if m is not None else {"w": gpu.tensor(np.ones(3, np.float32), device="gpu")}
    buf = io.BytesIO()
    S.save(sd, buf)
    rec = _Recorder(io.BytesIO(buf.getvalue()))
    rec.load()
    assert {p[6] for p in rec.pids if p[0] == "tensor_v3"} <= {"metal", "cpu"}
    back = S.load(io.BytesIO(buf.getvalue()))
    for k, v in sd.items():
        if hasattr(v, "numpy"):
            assert back[k].device == v.device
            np.testing.assert_array_equal(back[k].numpy(), v.numpy())


def test_sharded_checkpoints(tmp_path):
    """save_sharded / load_sharded (lucid/serialization/__init__.py:646-830): first-fit shards
    under the cap, a tensor over the cap alone, tied keys kept in one shard with the key order
    restored, the index layout, and the single-shard form of a non-dict object."""
    import json
    from collections import OrderedDict

    big = tensor(np.arange(300_000, dtype=np.float32))           # 1.14 MiB, over a 1 MiB cap
    w = tensor(np.ones((100, 100), np.float32))                   # 40 KB
    sd = OrderedDict([("a", tensor(np.arange(10, dtype=np.int8))), ("big", big), ("w", w),
                      ("c", tensor(np.float32(2.5))), ("tied", w)])
    sd._metadata = {"": {"version": 2}}
    d = tmp_path / "ckpt"
    S.save_sharded(sd, d, shard_size_mb=0.5)
    index = json.loads((d / "index.json").read_text())
    assert index["_lucid_sharded"] == 1 and index["_state_dict_metadata"] == {"": {"version": 2}}
    files = [e["file"] for e in index["shards"]]
    assert files == [f"shard-{i:05d}-of-{len(files):05d}.lucid" for i in range(len(files))]
    keysets = [e["keys"] for e in index["shards"]]
    assert ["big"] in keysets                                    # over the cap: a shard of its own
    assert any("w" in ks and "tied" in ks for ks in keysets)     # tied keys together
    assert index["key_order"] == list(sd)
    back = S.load_sharded(d)
    assert list(back) == list(sd) and back._metadata == {"": {"version": 2}}
    assert back["w"] is back["tied"]
    for k, v in sd.items():
        np.testing.assert_array_equal(back[k].numpy(), v.numpy())
    S.save_sharded([1, 2, big], tmp_path / "list")
    out = S.load_sharded(tmp_path / "list")
    assert out[:2] == [1, 2] and np.array_equal(out[2].numpy(), big.numpy())
    (tmp_path / "bad").mkdir()
    (tmp_path / "bad" / "index.json").write_text(json.dumps({"_lucid_sharded": 1, "shards": [
        {"file": "../x.lucid", "keys": ["a"]}]}))
    with pytest.raises(RuntimeError, match="plain file name"):
        S.load_sharded(tmp_path / "bad")
    with pytest.raises(TypeError):
        S.save_sharded(sd, big)
