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
