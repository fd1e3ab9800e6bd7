"""GPU parity of the LoRA adapters over the quantized linears (lucid_amd/peft, over the HIP
kernels): the forward pass against float64 (scale-aware rtol 1e-5) and bit-exact where it is
the base layer alone; merging into int8 / group-wise weights bit-exact against the oracle's
requantization of the same float32 merged weight (lucid/peft/tuners/lora/_weight_site.py:
162-243: per-channel symmetric qint8 min/max observer, the group quantizer); unmerge restores
the buffers bit for bit (_layer.py:1017-1046)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import assert_close_f32

pytestmark = pytest.mark.gpu


def _float_linear(L, W, b):
    import lucid_amd.nn as nn
    from lucid_amd.nn.module import Parameter

    lin = nn.Linear(W.shape[1], W.shape[0], bias=b is not None)
    lin.weight = Parameter(L.tensor(W, device="gpu"))
    if b is not None:
        lin.bias = Parameter(L.tensor(b, device="gpu"))
    return lin


def _random_factors(layer, rng, adapter="default"):
    """Give an adapter nonzero factors (as trained ones would be)."""
    from lucid_amd.nn.module import Parameter

    import lucid_amd as L

    a, b = layer.lora_A[adapter], layer.lora_B[adapter]
    a.weight = Parameter(L.tensor(rng.standard_normal(a.weight.shape).astype(np.float32) * 0.05, device="gpu"))
    b.weight = Parameter(L.tensor(rng.standard_normal(b.weight.shape).astype(np.float32) * 0.05, device="gpu"))
    return a.weight.numpy().astype(np.float64), b.weight.numpy().astype(np.float64)


def _bases(L, rng, K=256, N=192):
    """One base layer of each quantized type (and the float Linear), from the same float weight."""
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.nn.quantized.dynamic as nnqd
    import lucid_amd.quantization as Q
    import lucid_amd.nn as nn

    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    import lucid_amd.backends as backends

    static = nn.Sequential(nnq.QuantStub(), _float_linear(L, W, b), nnq.DeQuantStub())
    prepared = Q.prepare(static, Q.get_minmax_qconfig())
    for _ in range(3):
        prepared(L.tensor(rng.standard_normal((32, K)).astype(np.float32), device="gpu"))
    saved = backends.quantized.engine
    backends.quantized.engine = "reference"  # the int8 nnq.Linear, not the group-wise layer
    try:
        converted = Q.convert(prepared)
    finally:
        backends.quantized.engine = saved
    assert isinstance(converted[1], nnq.Linear)
    return {
        "float": _float_linear(L, W, b),
        "dynamic": nnqd.Linear.from_float(_float_linear(L, W, b)),
        "static": converted[1],
        "mlx4": nnq.QuantizedLinearMLX.from_float(_float_linear(L, W, b), bits=4, group_size=64),
    }


@pytest.mark.parametrize("kind", ["float", "dynamic", "static", "mlx4"])
def test_lora_forward(gpu, kind):
    """y = base(x) + s B A x: the base part bit for bit (B = 0 at creation: the layer is its
    base), the update within the scale-aware 1e-5 of float64."""
    from lucid_amd.peft import LoraConfig, lora_layer_for

    rng = np.random.default_rng({"float": 1, "dynamic": 2, "static": 3, "mlx4": 4}[kind])
    base = _bases(gpu, rng)[kind]
    K = base.in_features
    x = gpu.tensor(rng.standard_normal((9, K)).astype(np.float32), device="gpu")
    cfg = LoraConfig(r=8, lora_alpha=16, target_modules=["x"])
    layer = lora_layer_for(base, "default", cfg).eval()
    y0 = base(x).numpy()
    np.testing.assert_array_equal(layer(x).numpy(), y0)
    A, B = _random_factors(layer, rng)
    got = layer(x).numpy()
    upd = (x.numpy().astype(np.float64) @ A.T) @ B.T * cfg.scaling
    assert_close_f32(got - y0, upd)
    with_dis = layer
    with_dis.disable_adapters = True
    np.testing.assert_array_equal(with_dis(x).numpy(), y0)


@pytest.mark.parametrize("kind", ["dynamic", "static"])
def test_lora_merge_int8_exact(gpu, kind):
    """Merging into int8 codes: the codes, scales and zero points the per-channel symmetric
    observer and quantizer give for fl32(dequantize(W) + delta), bit for bit; unmerge restores
    the original buffers bit for bit."""
    from lucid_amd.peft import LoraConfig, lora_layer_for

    rng = np.random.default_rng(5)
    base = _bases(gpu, rng)[kind]
    cfg = LoraConfig(r=4, lora_alpha=8, target_modules=["x"])
    layer = lora_layer_for(base, "default", cfg).eval()
    A, B = _random_factors(layer, rng)
    before = {k: v.numpy().copy() for k, v in base._buffers.items() if v is not None}
    codes, s, z = before["weight_int8"], before["weight_scale"], before["weight_zero_point"]
    w_deq = O.dequantize(codes, O.I8, s, z, ch_axis=0)
    delta = layer.get_delta_weight("default").numpy()
    assert_close_f32(delta, (B @ A) * cfg.scaling)
    merged_w = (w_deq + delta).astype(np.float32)  # one float32 add, as the merge does
    mn, mx = O.minmax_per_channel(merged_w, 0)
    s2, z2 = O.calc_qparams(mn, mx, True, True, -128, 127)
    want = O.quantize(merged_w, O.recip_tensor(s2), z2, -128, 127, O.I8, ch_axis=0)
    layer.merge()
    np.testing.assert_array_equal(base.weight_int8.numpy(), want)
    np.testing.assert_array_equal(base.weight_scale.numpy().view(np.uint32), s2.view(np.uint32))
    np.testing.assert_array_equal(base.weight_zero_point.numpy(), z2)
    x = gpu.tensor(rng.standard_normal((5, base.in_features)).astype(np.float32), device="gpu")
    assert layer.merged and layer(x).numpy().shape == (5, base.out_features)  # the base alone now
    layer.unmerge()
    for k, v in before.items():
        np.testing.assert_array_equal(base._buffers[k].numpy(), v)
    assert not layer.merged


def test_lora_merge_group_wise_exact(gpu):
    """Merging into a group-wise 4-bit layer: the packed codes, scales and biases of the group
    quantizer for fl32(dequantize(W) + delta); unmerge restores them."""
    from lucid_amd.peft import LoraConfig, lora_layer_for

    rng = np.random.default_rng(9)
    base = _bases(gpu, rng)["mlx4"]
    layer = lora_layer_for(base, "default", LoraConfig(r=4, lora_alpha=4, target_modules=["x"])).eval()
    _random_factors(layer, rng)
    pw, sc, bi = base.packed_weight.numpy().copy(), base.scales.numpy().copy(), base.biases.numpy().copy()
    w_deq = O.group_dequantize(pw.view(np.uint32), sc, bi, 64, 4)
    merged_w = (w_deq + layer.get_delta_weight("default").numpy()).astype(np.float32)
    want = O.group_quantize(merged_w, 64, 4)
    layer.merge()
    np.testing.assert_array_equal(base.packed_weight.numpy().view(np.uint32), want[0].view(np.uint32))
    np.testing.assert_array_equal(base.scales.numpy().view(np.uint32), want[1].view(np.uint32))
    np.testing.assert_array_equal(base.biases.numpy().view(np.uint32), want[2].view(np.uint32))
    layer.unmerge()
    np.testing.assert_array_equal(base.packed_weight.numpy(), pw)
    np.testing.assert_array_equal(base.scales.numpy(), sc)


def test_peft_model_merge_and_unload(gpu):
    """get_peft_model over a dynamic-int8 MLP: merged output within the requantization error of
    the unmerged one; merge_and_unload hands back the base modules; the float Linear merge is
    the float sum."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.peft import LoraConfig, get_peft_model

    rng = np.random.default_rng(21)
    W1 = (rng.standard_normal((128, 64)) * 0.1).astype(np.float32)
    W2 = (rng.standard_normal((32, 128)) * 0.1).astype(np.float32)
    model = nn.Sequential(nnqd.Linear.from_float(_float_linear(gpu, W1, None)), nn.ReLU(),
                          _float_linear(gpu, W2, np.zeros(32, np.float32)))
    peft = get_peft_model(model, LoraConfig(r=4, lora_alpha=8, target_modules=["0", "2"])).eval()
    layers = [peft.base_model.model[0], peft.base_model.model[2]]
    for lay in layers:
        _random_factors(lay, rng)
    x = gpu.tensor(rng.standard_normal((6, 64)).astype(np.float32), device="gpu")
    y = peft(x).numpy()
    w2 = layers[1].base_layer.weight.numpy().copy()
    d2 = layers[1].get_delta_weight("default").numpy()
    peft.merge_adapter()
    np.testing.assert_array_equal(layers[1].base_layer.weight.numpy(), (w2 + d2).astype(np.float32))
    y_merged = peft(x).numpy()
    cos = float(np.sum(y * y_merged) / np.sqrt(np.sum(y * y) * np.sum(y_merged * y_merged)))
    assert cos > 0.999
    peft.unmerge_adapter()  # int8 buffers restored exactly, the float weight to within rounding
    assert_close_f32(peft(x).numpy(), y)
    plain = peft.merge_and_unload()
    assert isinstance(plain[0], nnqd.Linear) and isinstance(plain[2], nn.Linear)
    assert_close_f32(plain(x).numpy(), y_merged)
