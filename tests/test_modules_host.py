"""Host-side logic of the module layer (no GPU): config resolution, prepare's observer
wiring, fusion and the BatchNorm fold, the engine selector, state_dict layouts."""

from __future__ import annotations

import warnings

import numpy as np
import pytest


def _model():
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    return nn.Sequential(nnq.QuantStub(), nn.Linear(16, 8), nn.ReLU(), nn.Linear(8, 4),
                         nnq.DeQuantStub())


def test_qconfig_mapping_precedence():
    import lucid_amd.nn as nn
    from lucid_amd.quantization import QConfigMapping, get_default_qconfig, get_minmax_qconfig

    a, b = get_default_qconfig(), get_minmax_qconfig()
    m = QConfigMapping().set_global(a).set_object_type(nn.Linear, b).set_module_name("3", None)
    assert m.get_qconfig(nn.Linear, "1") is b
    assert m.get_qconfig(nn.Linear, "3") is None
    assert m.get_qconfig(nn.ReLU, "2") is a


def test_prepare_attaches_observers_and_hooks():
    import lucid_amd.nn as nn
    import lucid_amd.quantization as Q
    from lucid_amd.quantization.observer import MinMaxObserver

    model = _model()
    prepared = Q.prepare(model, Q.get_minmax_qconfig())
    assert prepared is not model
    for idx in ("0", "1", "3"):
        mod = getattr(prepared, idx)
        assert isinstance(mod.activation_post_process, MinMaxObserver)
        assert len(mod._forward_hooks) == 1
    assert not hasattr(prepared[2], "activation_post_process")
    assert isinstance(prepared[1], nn.Linear) and prepared.training is False
    # the observer buffers join the state dict under the module's prefix
    assert "1.activation_post_process.min_val" in prepared.state_dict()


def test_prepare_respects_none_and_warns_on_no_match():
    import lucid_amd.nn as nn
    import lucid_amd.quantization as Q

    model = _model()
    mapping = Q.QConfigMapping().set_global(Q.get_minmax_qconfig()).set_module_name("3", None)
    prepared = Q.prepare(model, mapping)
    assert hasattr(prepared[1], "activation_post_process")
    assert not hasattr(prepared[3], "activation_post_process")
    with pytest.warns(UserWarning, match="matched no quantizable modules"):
        Q.prepare(nn.Sequential(nn.ReLU()), Q.get_minmax_qconfig())
    with pytest.raises(TypeError):
        Q.prepare(model, qconfig="not a qconfig")


def test_fuse_linear_relu_and_identity_slots():
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.quantization as Q

    fused = Q.fuse_modules(_model(), [["1", "2"]])
    assert isinstance(fused[1], nni.LinearReLU) and isinstance(fused[2], nn.Identity)
    assert isinstance(fused[1][0], nn.Linear) and isinstance(fused[1][1], nn.ReLU)
    with pytest.raises(ValueError, match="unsupported fusion pattern"):
        Q.fuse_modules(_model(), [["2", "3"]])


def test_bn_fold_closed_form():
    """w' = w * gamma / sqrt(var + eps), b' = (b - mean) * gamma / sqrt(var + eps) + beta,
    against float64 (fusion.py:52-106; the reference checks the fold at atol 1e-4)."""
    import lucid_amd.nn as nn
    from lucid_amd._tensor import tensor
    from lucid_amd.quantization.fuse_modules import fuse_conv_bn_eval

    rng = np.random.default_rng(0)
    conv = nn.Conv2d(3, 6, 3)
    bn = nn.BatchNorm2d(6)
    bn.running_mean = tensor(rng.normal(0, 1, 6).astype(np.float32))
    bn.running_var = tensor(rng.uniform(0.5, 2, 6).astype(np.float32))
    bn.weight = nn.Parameter(tensor(rng.normal(1, 0.1, 6).astype(np.float32)))
    bn.bias = nn.Parameter(tensor(rng.normal(0, 0.1, 6).astype(np.float32)))
    conv.eval(), bn.eval()
    fused = fuse_conv_bn_eval(conv, bn)
    w = conv.weight.numpy().astype(np.float64)
    g = bn.weight.numpy() / np.sqrt(bn.running_var.numpy().astype(np.float64) + bn.eps)
    np.testing.assert_allclose(fused.weight.numpy(), w * g[:, None, None, None], rtol=1e-6)
    want_b = (conv.bias.numpy() - bn.running_mean.numpy()) * g + bn.bias.numpy()
    np.testing.assert_allclose(fused.bias.numpy(), want_b, rtol=1e-6, atol=1e-7)
    assert isinstance(fused, nn.Conv2d) and fused is not conv
    bn.train()
    with pytest.raises(AssertionError, match="eval"):
        fuse_conv_bn_eval(conv, bn)


def test_fuse_conv_bn_relu_run():
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.quantization as Q

    model = nn.Sequential(nn.Conv2d(3, 4, 3), nn.BatchNorm2d(4), nn.ReLU()).eval()
    fused = Q.fuse_modules(model, [["0", "1", "2"]])
    assert isinstance(fused[0], nni.ConvReLU2d)
    assert isinstance(fused[1], nn.Identity) and isinstance(fused[2], nn.Identity)


def test_engine_selector():
    import lucid_amd.backends as backends
    from lucid_amd.quantization._quantize import _mlx_group_size

    q = backends.quantized
    assert q.engine == "auto"
    with pytest.raises(ValueError):
        q.engine = "cuda"
    try:
        q.engine = "reference"
        assert q.use_mlx() is False
        q.engine = "mlx_group"
        assert q.use_mlx() is True
    finally:
        q.engine = "auto"
    assert _mlx_group_size(784) is None and _mlx_group_size(256) == 64
    assert _mlx_group_size(128 + 256) == 64 and _mlx_group_size(96) == 32
    assert _mlx_group_size(128 * 3) == 64


def test_dynamic_spec_normalisation():
    import lucid_amd.nn as nn
    from lucid_amd.quantization import qint8
    from lucid_amd.quantization._propagate import dynamic_rules, weight_dtype

    mapping, labels = dynamic_rules({nn.Linear: qint8, "head": None}, qint8, (nn.Linear,))
    assert labels == ("Linear",)
    assert mapping.get_qconfig(nn.Linear, "x") is not None
    assert mapping.get_qconfig(nn.Linear, "head") is None
    assert weight_dtype(mapping.get_qconfig(nn.Linear, "x"), None) is qint8
    with pytest.raises(TypeError, match="qconfig_spec must be"):
        dynamic_rules("Linear", qint8, (nn.Linear,))
    with pytest.raises(TypeError, match="keys must be"):
        dynamic_rules({3: qint8}, qint8, (nn.Linear,))
    with pytest.raises(TypeError, match=r"qconfig_spec\['head'\] must be"):
        dynamic_rules({"head": 3.0}, qint8, (nn.Linear,))


def test_resolution_tiers_and_inheritance():
    """Own .qconfig > name rule > type rule > parent; the root takes the global recipe, except
    under the stock default when the user has configured modules."""
    import lucid_amd.nn as nn
    import lucid_amd.quantization as Q
    from lucid_amd.quantization._propagate import plan_sites

    a, b = Q.get_minmax_qconfig(), Q.get_default_qconfig()
    inner = nn.Sequential(nn.Linear(4, 4), nn.ReLU())
    model = nn.Sequential(nn.Linear(4, 4), inner, nn.Linear(4, 2))
    mapping = Q.QConfigMapping().set_global(a).set_object_type(nn.ReLU, None).set_module_name("2", b)
    got = {s.path: s.qconfig for s in plan_sites(model, mapping)}
    assert got[""] is a and got["0"] is a and got["1"] is a and got["1.0"] is a
    assert got["1.1"] is None and got["2"] is b
    # a name rule beats a type rule for the same module
    mapping.set_object_type(nn.Linear, None)
    got = {s.path: s.qconfig for s in plan_sites(model, mapping)}
    assert got["0"] is None and got["1.0"] is None and got["2"] is b
    # a module's own attribute beats both; its children inherit it
    inner.qconfig = b
    got = {s.path: s.qconfig for s in plan_sites(model, Q.QConfigMapping().set_global(a))}
    assert got["1"] is b and got["1.0"] is b and got["0"] is a
    # the stock default does not fill in around user-configured modules
    got = {s.path: s.qconfig for s in plan_sites(model, Q.QConfigMapping().set_global(a), stock_default=True)}
    assert got[""] is None and got["0"] is None and got["1"] is b
    del inner.qconfig
    # a module shared along two paths is planned once, at its first occurrence
    shared = nn.Linear(4, 4)
    twice = nn.Sequential(shared, nn.Sequential(shared))
    paths = [s.path for s in plan_sites(twice, Q.QConfigMapping())]
    assert paths == ["", "0", "1"]
    with pytest.raises(TypeError, match="qconfig must be a QConfig or None"):
        inner.qconfig = "x"
        plan_sites(model, Q.QConfigMapping())


def test_quantize_dynamic_replacement_and_warnings():
    """The dynamic swap's walk with stand-in builders (no GPU): the root itself may be
    replaced; nested targets are; a replaced module's subtree is left alone; a named leaf
    without a dynamic form warns that it stays float; nothing targeted warns the model is
    unchanged."""
    import lucid_amd.nn as nn
    from lucid_amd.nn.module import Module
    from lucid_amd.quantization import qint8
    from lucid_amd.quantization._propagate import dynamic_rules
    from lucid_amd.quantization._quantize import _replace_dynamic

    class Swapped(Module):
        def __init__(self, src, dtype):
            super().__init__()
            self.src, self.dtype = src, dtype

    class Block(Module):  # a container type with a builder: replaced whole
        def __init__(self):
            super().__init__()
            self.lin = nn.Linear(8, 8)

    builders = {nn.Linear: Swapped, Block: Swapped}

    def run(model, spec):
        mapping, labels = dynamic_rules(spec, qint8, tuple(builders))
        return _replace_dynamic(model, mapping, labels, builders, qint8)

    root = nn.Linear(8, 4)
    assert isinstance(run(root, None), Swapped)
    model = nn.Sequential(nn.Linear(8, 8), nn.Sequential(nn.ReLU(), nn.Linear(8, 4)), Block())
    out = run(model, {nn.Linear, Block})
    assert out is model and isinstance(model[0], Swapped) and isinstance(model[1][1], Swapped)
    assert isinstance(model[2], Swapped) and isinstance(model[2].src.lin, nn.Linear)  # subtree kept
    model = nn.Sequential(nn.Linear(8, 8), nn.Sequential(nn.ReLU(), nn.Linear(8, 4)))
    run(model, {"1.1": None, nn.Linear: qint8})  # a name rule beats the type rule
    assert isinstance(model[0], Swapped) and isinstance(model[1][1], nn.Linear)
    with pytest.warns(UserWarning, match="ReLU has no dynamically quantized form"):
        run(nn.Sequential(nn.ReLU(), nn.Linear(2, 2)), {nn.ReLU})
    with pytest.warns(UserWarning, match=r"no module of a targeted type \(Conv2d\) found"):
        run(nn.Sequential(nn.ReLU()), {nn.Conv2d})
    # a Linear tied at two places (the reference's swap walks every parent slot,
    # lucid/quantization/_quantize.py:588-602): both slots are swapped, to one quantized module
    shared = nn.Linear(4, 4)
    tied = nn.Sequential(shared, nn.ReLU(), shared, nn.Sequential(shared))
    run(tied, {nn.Linear})
    assert isinstance(tied[0], Swapped) and tied[2] is tied[0] and tied[3][0] is tied[0]
    assert tied[0].src is shared
    # a tied layer excluded by name at one place stays float only there
    shared = nn.Linear(4, 4)
    tied = nn.Sequential(shared, shared)
    run(tied, {"1": None, nn.Linear: qint8})
    assert isinstance(tied[0], Swapped) and tied[1] is shared


def test_quantized_module_state_dict_layouts():
    """Lucid's buffer names, dtypes and shapes (lucid/nn/quantized/linear.py:190-203,
    dynamic/linear.py:68-83, modules.py:229-278)."""
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.nn.quantized.dynamic as nnqd

    sd = nnq.Linear(16, 8).state_dict()
    assert list(sd) == ["weight_int8", "weight_scale", "weight_zero_point", "bias", "scale",
                        "zero_point"]
    assert sd["weight_int8"].dtype == np.int8 and sd["weight_int8"].shape == (8, 16)
    assert sd["weight_scale"].dtype == np.float32 and sd["weight_scale"].shape == (8,)
    assert sd["scale"].shape == () and sd["zero_point"].shape == ()
    assert "bias" not in nnq.Linear(16, 8, bias=False).state_dict()
    assert list(nnqd.Linear(16, 8).state_dict()) == ["weight_int8", "weight_scale",
                                                     "weight_zero_point", "bias"]
    assert list(nnq.Quantize(0.1, 3).state_dict()) == ["scale", "zero_point"]
    assert nnq.DeQuantize().state_dict() == {}
    w = nnq.QuantWrapper(nnq.Linear(4, 2))
    assert [n for n, _ in w.named_children()] == ["quant", "module", "dequant"]


def test_quantized_ops_refuse_cpu_tensors():
    """No CPU fallback: the quantized modules raise on host tensors."""
    import lucid_amd as L
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.nn.quantized.dynamic as nnqd

    x = L.tensor(np.zeros((2, 16), np.float32))
    for mod in (nnq.Linear(16, 8), nnqd.Linear(16, 8)):
        with pytest.raises(L.LucidError, match="GPU"):
            mod(x)


def test_stubs_are_identity_before_prepare():
    import lucid_amd as L
    import lucid_amd.nn.quantized as nnq

    x = L.tensor(np.arange(3, dtype=np.float32))
    assert nnq.QuantStub()(x) is x and nnq.DeQuantStub()(x) is x and nnq.DeQuantize()(x) is x
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert nnq.Quantize(0.1, 0)(L.tensor(np.arange(3, dtype=np.int32))).dtype == np.int32


def test_group_ops_reject_mismatched_operands_before_launch():
    """quantized_matmul / dequantize validate the packed weight, scales and biases on the host
    (a scale table built for another group size would be read past its end on the device)."""
    import lucid_amd as L
    from lucid_amd.quantization import _qgemm

    N, K = 8, 256
    wq = L.tensor(np.zeros((N, K * 4 // 32), np.int32))  # 4-bit codes of an 8 x 256 weight
    s64 = L.tensor(np.ones((N, K // 64), np.float32))
    b64 = L.tensor(np.zeros((N, K // 64), np.float32))
    x = L.tensor(np.zeros((2, K), np.float32))
    # scales of group size 64 used with group size 32: refused, not read out of bounds
    with pytest.raises(ValueError, match="scales must be"):
        _qgemm.quantized_matmul(x, wq, s64, b64, group_size=32, bits=4)
    with pytest.raises(ValueError, match="scales must be"):
        _qgemm.dequantize(wq, s64, b64, group_size=32, bits=4)
    with pytest.raises(ValueError, match="biases must be"):
        _qgemm.quantized_matmul(x, wq, s64, L.tensor(np.zeros((N, 2), np.float32)), group_size=64, bits=4)
    with pytest.raises(ValueError, match="scales must be"):
        _qgemm.quantized_matmul(x, wq, L.tensor(np.ones((N + 1, K // 64), np.float32)), b64,
                                group_size=64, bits=4)
    with pytest.raises(TypeError, match="2-D int32"):
        _qgemm.quantized_matmul(x, L.tensor(np.zeros((N, 2, 16), np.int32)), s64, b64, bits=4)
    with pytest.raises(TypeError, match="2-D int32"):
        _qgemm.dequantize(L.tensor(np.zeros((N, 32), np.float32)), s64, b64, bits=4)
    with pytest.raises(ValueError, match="bias must be"):
        _qgemm.quantized_matmul(x, wq, s64, b64, group_size=64, bits=4,
                                bias=L.tensor(np.zeros(N + 1, np.float32)))
    with pytest.raises(ValueError, match="group_size must be"):
        _qgemm.quantized_matmul(x, wq, s64, b64, group_size=48, bits=4)
    # well-formed operands get as far as the device requirement
    with pytest.raises(L.LucidError, match="GPU"):
        _qgemm.quantized_matmul(x, wq, s64, b64, group_size=64, bits=4)


def test_fuse_conv1d_conv3d_bn_relu():
    """[Conv1d, BatchNorm1d, ReLU] and [Conv3d, BatchNorm3d] fold the BN into the conv (the
    closed form of lucid/nn/utils/fusion.py:52-106 over any kernel rank); the 1-D run becomes
    ConvReLU1d, a BatchNorm of the wrong rank is not fused."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    from lucid_amd._tensor import tensor
    from lucid_amd.quantization import fuse_modules

    rng = np.random.default_rng(0)
    for conv, bn, relu in ((nn.Conv1d(3, 4, 3), nn.BatchNorm1d(4), True), (nn.Conv3d(3, 4, 3), nn.BatchNorm3d(4), False)):
        bn.running_mean = tensor(rng.standard_normal(4).astype(np.float32))
        bn.running_var = tensor(rng.uniform(0.5, 2, 4).astype(np.float32))
        mods = [conv, bn] + ([nn.ReLU()] if relu else [])
        model = nn.Sequential(*mods).eval()
        fused = fuse_modules(model, [[str(i) for i in range(len(mods))]])
        head = fused[0]
        assert isinstance(head, nni.ConvReLU1d) if relu else type(head) is nn.Conv3d
        inner = head[0] if relu else head
        w = conv.weight.numpy()
        scale = (1.0 / np.sqrt(bn.running_var.numpy() + np.float32(bn.eps))).astype(np.float32)
        want = (w * scale.reshape((-1,) + (1,) * (w.ndim - 1))).astype(np.float32)
        np.testing.assert_array_equal(inner.weight.numpy(), want)
    with pytest.raises(ValueError, match="unsupported"):
        fuse_modules(nn.Sequential(nn.BatchNorm1d(4), nn.Conv1d(4, 4, 1)).eval(), [["0", "1"]])


def test_conv_nd_modules_map_and_keep_state_dict_layout():
    """convert's table covers the 1-D / 3-D family; the quantized modules keep Lucid's buffer
    names and shapes (weight_int8 [out, in / groups, *k], transposed [in, out / groups, *k])."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.quantization._quantize import _observed_types, _quant_mapping

    mapping = _quant_mapping()
    for t in (nn.Conv1d, nn.Conv3d, nn.ConvTranspose1d, nn.ConvTranspose3d, nni.ConvReLU1d, nni.ConvReLU3d):
        assert t in mapping and t in _observed_types()
    sd = nnq.Conv3d(4, 8, (3, 2, 1), groups=2).state_dict()
    assert sd["weight_int8"].shape == (8, 2, 3, 2, 1) and sd["weight_scale"].shape == (8,)
    sd = nnq.ConvTranspose3d(4, 6, 3, groups=2).state_dict()
    assert sd["weight_int8"].shape == (4, 3, 3, 3, 3) and sd["weight_scale"].shape == (3,)
    assert set(nnq.Conv1d(2, 3, 5).state_dict()) == {"weight_int8", "weight_scale", "weight_zero_point", "bias",
                                                      "scale", "zero_point"}


def test_packed_sequence_validation():
    """PackedSequence checks its batch sizes and derives the inverse permutation
    (lucid/nn/utils/rnn.py:140-150, 184-260)."""
    from lucid_amd._tensor import tensor
    from lucid_amd.nn.utils.rnn import PackedSequence

    data = tensor(np.zeros((3, 2), np.float32))
    p = PackedSequence(data, [2, 1], [1, 0])
    assert p.unsorted_indices.numpy().tolist() == [1, 0]
    assert p.batch_sizes.numpy().dtype == np.int64
    data, bs, si, ui = p  # a 4-tuple
    with pytest.raises(ValueError, match="non-increasing"):
        PackedSequence(data, [1, 2])
    with pytest.raises(ValueError, match="sums to"):
        PackedSequence(data, [2, 2])
    with pytest.raises(ValueError, match="permutation"):
        PackedSequence(data, [2, 1], [0, 0])


def test_conv_size_arguments_refuse_wrong_lengths():
    """A convolution's size arguments are read as Lucid reads them (nn/modules/_conv_common.py:16,
    nn/functional/_spatial_args.py:28): an int or a sequence of one repeats, a sequence of the
    rank is taken, any other length raises -- and a kernel_size must name every axis."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.nn.functional import _ntuple

    assert _ntuple(3, 3) == (3, 3, 3) and _ntuple([2], 3, "stride") == (2, 2, 2)
    assert _ntuple((1, 2, 3), 3, "kernel_size") == (1, 2, 3)
    for bad, name in (((3, 5), "kernel_size"), ([2, 2, 2, 2], "stride"), ((3,), "kernel_size")):
        with pytest.raises(ValueError, match=name):
            _ntuple(bad, 3, name)
    with pytest.raises(ValueError, match="kernel_size"):
        nn.Conv3d(2, 2, kernel_size=(3, 5))
    with pytest.raises(ValueError, match="stride"):
        nn.Conv1d(2, 2, 3, stride=(1, 2))
    with pytest.raises(ValueError, match="padding"):
        nnq.Conv3d(2, 2, 3, padding=(1, 1))
    assert nn.Conv3d(2, 2, 3, stride=[2]).stride == (2, 2, 2)


def test_lstm_projection_parameters_and_refusals():
    """proj_size registers weight_hr_l{k}[_reverse] [P, H] after each layer's biases, shrinks
    weight_hh to [4H, P] and a deeper layer's weight_ih to [4H, D P], and is refused as the
    reference refuses it (lucid/nn/modules/recurrent_base.py:138-145, 164-194)."""
    import lucid_amd.nn as nn

    m = nn.LSTM(4, 6, num_layers=2, bidirectional=True, proj_size=2)
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    names = list(shapes)
    assert names[:6] == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "weight_hr_l0",
                         "weight_ih_l0_reverse"]
    assert shapes["weight_hh_l0"] == (24, 2) and shapes["weight_hr_l1_reverse"] == (2, 6)
    assert shapes["weight_ih_l1"] == (24, 4)
    assert "proj_size=2" in repr(m)
    assert "weight_hr_l0" not in dict(nn.LSTM(4, 6).named_parameters())
    for bad in (6, 7, -1):
        with pytest.raises(ValueError):
            nn.LSTM(4, 6, proj_size=bad)
