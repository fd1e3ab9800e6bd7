"""lucid_amd.graphs.CapturedForward: a module forward recorded once and replayed as one HIP
graph gives the eager forward's bits, for new inputs loaded into the captured buffers, at
BASELINE configurations 1 (dynamic int8 MLP) and 5 (static int8 ResNet-18, batch 2); calls a
graph cannot replay are refused while recording."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture
def reference_engine():
    """Per-channel int8 Linears (the configurations' layers), not the group-wise engine."""
    import lucid_amd.backends as backends

    backends.quantized.engine = "reference"
    yield
    backends.quantized.engine = "auto"


def _same(a, b):
    np.testing.assert_array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


def test_mlp_replay_is_the_eager_forward(gpu, reference_engine):
    import lucid_amd.nn as nn
    from lucid_amd.graphs import CapturedForward
    from lucid_amd.quantization import quantize_dynamic

    rng = np.random.default_rng(5)
    lins = []
    for k, n in ((784, 256), (256, 10)):
        m = nn.Linear(k, n)
        m.weight = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, (n, k)).astype(np.float32)))
        m.bias = nn.Parameter(gpu.tensor(rng.normal(0, 0.05, n).astype(np.float32)))
        lins.append(m)
    q = quantize_dynamic(nn.Sequential(lins[0], nn.ReLU(), lins[1]))
    x = gpu.tensor(rng.standard_normal((64, 784)).astype(np.float32), device="gpu")
    want = q(x).numpy()
    cap = CapturedForward(q, x)
    assert cap.launches >= 4
    for _ in range(3):
        _same(cap().numpy(), want)
    x2 = rng.standard_normal((64, 784)).astype(np.float32) * 3
    cap.load(x2)
    got = cap().numpy()
    _same(got, q(gpu.tensor(x2, device="gpu")).numpy())


def test_resnet18_replay_is_the_eager_forward(gpu, reference_engine):
    from lucid_amd.bench_configs import static_resnet18
    from lucid_amd.graphs import CapturedForward

    qnet, x = static_resnet18(batch=2, calib_batches=2)
    want = qnet(x).numpy()
    cap = CapturedForward(qnet, x)
    _same(cap().numpy(), want)
    rng = np.random.default_rng(9)
    x2 = rng.standard_normal(tuple(x.shape)).astype(np.float32)
    cap.load(x2)
    got = cap().numpy()
    _same(got, qnet(gpu.tensor(x2, device="gpu")).numpy())
    _same(cap().numpy(), got)  # replays again from the same input


def test_unreplayable_calls_are_refused(gpu):
    from lucid_amd import _C
    from lucid_amd.graphs import CaptureError, CapturedForward

    y = gpu.empty((16,), np.float32, "gpu")

    def uploads():
        gpu.tensor(np.arange(16, dtype=np.float32), device="gpu")  # a host -> device copy
        return y

    with pytest.raises(CaptureError, match="lq_memcpy_h2d"):
        CapturedForward(uploads, warmup=0)

    def own_stream():
        _C.call("lq_fill_u32", y.data_ptr(), 0, 16, cap_stream.value)
        return y

    import ctypes

    cap_stream = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(cap_stream))
    try:
        with pytest.raises(CaptureError, match="stream of its own"):
            CapturedForward(own_stream, warmup=0)
    finally:
        _C.call("lq_stream_destroy", cap_stream)


@pytest.mark.parametrize("batch", [2, 32])
def test_resnet18_nhwc_runtime_is_the_module_forward(gpu, reference_engine, batch):
    """Int8ResNet (activations padded NHWC between the block convolutions, the residual adds
    fused into the second convolutions) gives the module forward's bits, eagerly and replayed
    as one graph, for two inputs."""
    from lucid_amd.bench_configs import Int8ResNet, static_resnet18
    from lucid_amd.graphs import CapturedForward

    qnet, x = static_resnet18(batch=batch, calib_batches=2)
    rt = Int8ResNet(qnet, batch)
    _same(rt(x).numpy(), qnet(x).numpy())
    cap = CapturedForward(rt, x)
    rng = np.random.default_rng(batch)
    for _ in range(2):
        x2 = rng.standard_normal(tuple(x.shape)).astype(np.float32)
        cap.load(x2)
        _same(cap().numpy(), qnet(gpu.tensor(x2, device="gpu")).numpy())
