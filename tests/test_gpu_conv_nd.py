"""GPU parity of the 1-D / 3-D convolutions and transposed convolutions (lucid_amd/nn/
quantized/conv_nd.py, lucid_amd/nn/functional.py over lq_depth_gather / lq_permute_0213 and the
2-D kernels).

References here are the direct definitions, written independently of the gather: the
windowed sum y[n, o, p] = sum_{c, k} x[n, c, p s - pad + k d] w[o, c, k] over a padded
input, and the transposed convolution's scatter y[n, o, i s - pad + k d] += x[n, c, i] w[c, o, k]
(lucid/nn/functional/conv.py; Conv.cpp:271-360).  int8 layers: the int32 sums exact, then the
oracle's W8A8 epilogue -> the output codes bit-exact (conv.py:126-134).  Float paths within the
scale-aware rtol 1e-5 of float64."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import assert_close_f32

pytestmark = pytest.mark.gpu


def conv_nd_direct(x, w, stride, pads, dil, groups, mode="zeros"):
    """x [N, C, *sp] (int64 or float64), w [Cout, C / groups, *k]; pads [(before, after)] per axis."""
    N, C = x.shape[:2]
    nd = x.ndim - 2
    Cout, Cg = w.shape[:2]
    ks = w.shape[2:]
    np_mode = {"zeros": "constant", "reflect": "reflect", "replicate": "edge", "circular": "wrap"}[mode]
    xp = np.pad(x, [(0, 0), (0, 0)] + list(pads), mode=np_mode)
    out = [(x.shape[2 + i] + pads[i][0] + pads[i][1] - dil[i] * (ks[i] - 1) - 1) // stride[i] + 1 for i in range(nd)]
    y = np.zeros((N, Cout, *out), x.dtype)
    og = Cout // groups
    for g in range(groups):
        xs = xp[:, g * Cg:(g + 1) * Cg]
        for kidx in np.ndindex(*ks):
            sl = tuple(slice(kidx[i] * dil[i], kidx[i] * dil[i] + stride[i] * (out[i] - 1) + 1, stride[i])
                       for i in range(nd))
            patch = xs[(slice(None), slice(None)) + sl]
            wk = w[(slice(g * og, (g + 1) * og), slice(None)) + kidx]
            y[:, g * og:(g + 1) * og] += np.einsum("nc...,oc->no...", patch, wk)
    return y


def conv_transpose_nd_direct(x, w, stride, pad, out_pad, dil, groups):
    """x [N, Cin, *sp], w [Cin, Cout / groups, *k]: the scatter definition, cropped by pad."""
    N, Cin = x.shape[:2]
    nd = x.ndim - 2
    Cog = w.shape[1]
    ks = w.shape[2:]
    sp = x.shape[2:]
    full = [(sp[i] - 1) * stride[i] + dil[i] * (ks[i] - 1) + 1 + out_pad[i] for i in range(nd)]
    y = np.zeros((N, Cog * groups, *full), x.dtype)
    cg = Cin // groups
    for g in range(groups):
        xs = x[:, g * cg:(g + 1) * cg]
        for kidx in np.ndindex(*ks):
            sl = tuple(slice(kidx[i] * dil[i], kidx[i] * dil[i] + stride[i] * (sp[i] - 1) + 1, stride[i])
                       for i in range(nd))
            wk = w[(slice(g * cg, (g + 1) * cg), slice(None)) + kidx]
            y[(slice(None), slice(g * Cog, (g + 1) * Cog)) + sl] += np.einsum("nc...,co->no...", xs, wk)
    out = [(sp[i] - 1) * stride[i] - 2 * pad[i] + dil[i] * (ks[i] - 1) + out_pad[i] + 1 for i in range(nd)]
    return y[(slice(None), slice(None)) + tuple(slice(pad[i], pad[i] + out[i]) for i in range(nd))]


def _code_input(L, rng, shape, scale=0.03, zp=117.0):
    """A code-backed input on the uint8 grid (codes stored as c - 128)."""
    from lucid_amd._tensor import QuantSource, Tensor

    c = rng.integers(0, 256, shape).astype(np.int64)
    codes = L.tensor((c - 128).astype(np.int8), device="gpu")
    q = QuantSource(codes, __import__("lucid_amd")._C.U8S8, L.tensor(np.float32(scale), device="gpu"),
                    L.tensor(np.float32(zp), device="gpu"), 0, 255)
    return Tensor._code_backed(q, shape), c, np.float32(scale), np.float32(zp)


def _set_int8(mod, rng, L, axis=0, relu=False):
    """Random symmetric per-channel int8 weights, bias and an output grid on the module."""
    w = rng.integers(-127, 128, tuple(mod.weight_int8.shape)).astype(np.int8)
    n = w.shape[axis]
    mod.register_buffer("weight_int8", L.tensor(w, device="gpu"))
    mod.register_buffer("weight_scale", L.tensor(rng.uniform(2e-3, 8e-3, n).astype(np.float32), device="gpu"))
    mod.register_buffer("weight_zero_point", L.tensor(np.zeros(n, np.float32), device="gpu"))
    if mod.bias is not None:
        mod.register_buffer("bias", L.tensor(rng.standard_normal(mod.out_channels).astype(np.float32) * 0.3,
                                             device="gpu"))
    mod.register_buffer("scale", L.tensor(np.float32(0.05), device="gpu"))
    mod.register_buffer("zero_point", L.tensor(np.float32(100.0), device="gpu"))
    return w


def _expected_codes(acc, x_scale, mod, channels_last_shape, relu):
    """The oracle's epilogue over acc [N, Cout, *out] -> uint8-grid codes in NC* order (as c - 128)."""
    N, Cout = acc.shape[:2]
    flat = np.moveaxis(acc, 1, -1).reshape(-1, Cout)
    ws = mod.weight_scale.numpy().reshape(-1)
    if ws.size != Cout:  # transposed layers: per (group, channel)
        ws = np.tile(ws, Cout // ws.size)
    b = mod.bias.numpy() if mod.bias is not None else None
    y = O.gemm_epilogue(flat.astype(np.int32), x_scale, ws, b, float(mod.scale.numpy()),
                        float(mod.zero_point.numpy()), 0, 255, O.OUT_QU8S8, relu)
    return np.moveaxis(y.reshape(N, *acc.shape[2:], Cout), -1, 1)


CONV3D_CASES = [  # (N, C, D, H, W, Cout, k, stride, pad, dil, groups, mode)
    (2, 8, 5, 9, 10, 16, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 1, "zeros"),
    (1, 16, 6, 7, 7, 32, (3, 2, 3), (2, 1, 2), (1, 0, 1), (1, 1, 1), 2, "zeros"),
    (2, 4, 7, 6, 5, 8, (2, 3, 3), (1, 2, 1), (0, 1, 1), (2, 1, 1), 1, "zeros"),
    (1, 8, 4, 6, 6, 8, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 1, "reflect"),
    (1, 8, 4, 5, 6, 8, (3, 1, 3), (1, 1, 1), (2, 0, 1), (1, 1, 1), 1, "replicate"),
    (2, 8, 5, 5, 5, 16, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 4, "circular"),
]


@pytest.mark.parametrize("case", CONV3D_CASES)
@pytest.mark.parametrize("relu", [False, True])
def test_quantized_conv3d_exact(gpu, case, relu):
    import lucid_amd.nn.quantized as nnq

    N, C, D, H, W, Cout, k, s, p, d, g, mode = case
    print(f"conv3d {case} relu={relu}", flush=True)
    rng = np.random.default_rng(sum(case[:6]) + relu)
    mod = (nnq.ConvReLU3d if relu else nnq.Conv3d)(C, Cout, k, s, p, d, g)
    mod.padding_mode = mode
    w = _set_int8(mod, rng, gpu)
    x, c, xs, xz = _code_input(gpu, rng, (N, C, D, H, W))
    y = mod(x)
    acc = conv_nd_direct(c - int(xz), w.astype(np.int64), s, [(v, v) for v in p], d, g, mode)
    want = _expected_codes(acc, xs, mod, None, relu)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)


@pytest.mark.parametrize("case", [(2, 8, 50, 16, 3, 1, 1, 1, 1), (3, 16, 33, 32, 5, 2, 2, 1, 4),
                                  (1, 4, 40, 8, 3, 1, 2, 3, 1), (2, 8, 20, 8, 4, 3, 0, 1, 2)])
def test_quantized_conv1d_exact(gpu, case):
    import lucid_amd.nn.quantized as nnq

    N, C, Lx, Cout, k, s, p, d, g = case
    rng = np.random.default_rng(sum(case))
    mod = nnq.Conv1d(C, Cout, k, s, p, d, g)
    w = _set_int8(mod, rng, gpu)
    x, c, xs, xz = _code_input(gpu, rng, (N, C, Lx))
    y = mod(x)
    acc = conv_nd_direct(c - int(xz), w.astype(np.int64), (s,), [(p, p)], (d,), g)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), _expected_codes(acc, xs, mod, None, False))


@pytest.mark.parametrize("case", [  # (N, Cin, sp, Cout, k, stride, pad, out_pad, dil, groups)
    (2, 8, (4, 5, 6), 16, (3, 3, 3), (2, 2, 2), (1, 1, 1), (1, 0, 1), (1, 1, 1), 1),
    (1, 16, (3, 4, 4), 8, (2, 3, 2), (1, 2, 2), (0, 1, 0), (0, 1, 1), (1, 1, 1), 2),
    (2, 4, (5, 3, 4), 4, (3, 2, 3), (3, 1, 2), (1, 0, 2), (2, 0, 0), (1, 1, 2), 1),
])
def test_quantized_conv_transpose3d_exact(gpu, case):
    import lucid_amd.nn.quantized as nnq

    N, Cin, sp, Cout, k, s, p, op, d, g = case
    print(f"convt3d {case}", flush=True)
    rng = np.random.default_rng(sum(sp) + Cin + Cout)
    mod = nnq.ConvTranspose3d(Cin, Cout, k, s, p, op, d, g)
    w = _set_int8(mod, rng, gpu, axis=1)
    x, c, xs, xz = _code_input(gpu, rng, (N, Cin, *sp))
    y = mod(x)
    acc = conv_transpose_nd_direct(c - int(xz), w.astype(np.int64), s, p, op, d, g)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), _expected_codes(acc, xs, mod, None, False))


@pytest.mark.parametrize("case", [(2, 8, 9, 16, 3, 2, 1, 1, 1, 1), (1, 8, 12, 8, 4, 3, 1, 2, 1, 2)])
def test_quantized_conv_transpose1d_exact(gpu, case):
    import lucid_amd.nn.quantized as nnq

    N, Cin, Lx, Cout, k, s, p, op, d, g = case
    rng = np.random.default_rng(sum(case))
    mod = nnq.ConvTranspose1d(Cin, Cout, k, s, p, op, d, g)
    w = _set_int8(mod, rng, gpu, axis=1)
    x, c, xs, xz = _code_input(gpu, rng, (N, Cin, Lx))
    y = mod(x)
    acc = conv_transpose_nd_direct(c - int(xz), w.astype(np.int64), (s,), (p,), (op,), (d,), g)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), _expected_codes(acc, xs, mod, None, False))


def test_float_conv_family(gpu):
    """F.conv1d / conv3d / conv_transpose1d / conv_transpose3d against float64 direct sums."""
    from lucid_amd.nn import functional as F

    rng = np.random.default_rng(4)
    x3 = rng.standard_normal((2, 6, 5, 7, 6)).astype(np.float32)
    w3 = rng.standard_normal((8, 3, 3, 2, 3)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    got = F.conv3d(gpu.tensor(x3, device="gpu"), gpu.tensor(w3, device="gpu"), gpu.tensor(b, device="gpu"),
                   (2, 1, 1), (1, 0, 1), (1, 2, 1), 2, "reflect").numpy()
    want = conv_nd_direct(x3.astype(np.float64), w3.astype(np.float64), (2, 1, 1), [(1, 1), (0, 0), (1, 1)],
                          (1, 2, 1), 2, "reflect") + b.reshape(1, -1, 1, 1, 1)
    assert_close_f32(got, want)
    x1 = rng.standard_normal((3, 4, 30)).astype(np.float32)
    w1 = rng.standard_normal((6, 4, 5)).astype(np.float32)
    got = F.conv1d(gpu.tensor(x1, device="gpu"), gpu.tensor(w1, device="gpu"), None, 2, 2, 1,
                   1).numpy()
    assert_close_f32(got, conv_nd_direct(x1.astype(np.float64), w1.astype(np.float64), (2,), [(2, 2)], (1,), 1))
    wt = rng.standard_normal((6, 2, 3, 3, 2)).astype(np.float32)  # [Cin, Cout/groups, k]
    got = F.conv_transpose3d(gpu.tensor(x3, device="gpu"), gpu.tensor(wt, device="gpu"), None, (2, 1, 2),
                             (1, 1, 0), (1, 0, 1), 3, 1).numpy()
    assert_close_f32(got, conv_transpose_nd_direct(x3.astype(np.float64), wt.astype(np.float64), (2, 1, 2),
                                                   (1, 1, 0), (1, 0, 1), (1, 1, 1), 3))
    wt1 = rng.standard_normal((4, 3, 4)).astype(np.float32)
    got = F.conv_transpose1d(gpu.tensor(x1, device="gpu"), gpu.tensor(wt1, device="gpu"), None, 3, 1, 2, 1,
                             1).numpy()
    assert_close_f32(got, conv_transpose_nd_direct(x1.astype(np.float64), wt1.astype(np.float64), (3,), (1,), (2,),
                                                   (1,), 1))


def test_static_ptq_conv3d_pipeline(gpu):
    """fuse [Conv3d, BatchNorm3d, ReLU] -> prepare -> calibrate -> convert gives ConvReLU3d whose
    codes are the direct int8 definition over its own buffers, and a Conv1d stack likewise."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.quantization as Q

    rng = np.random.default_rng(8)
    model = nn.Sequential(nnq.QuantStub(), nn.Conv3d(4, 8, 3, 1, 1), nn.BatchNorm3d(8), nn.ReLU(),
                          nnq.DeQuantStub())
    bn = model[2]
    bn.running_mean = gpu.tensor(rng.standard_normal(8).astype(np.float32) * 0.1)
    bn.running_var = gpu.tensor(rng.uniform(0.5, 2.0, 8).astype(np.float32))
    model.eval()
    model = Q.fuse_modules(model, [["1", "2", "3"]])
    assert type(model[1]).__name__ == "ConvReLU3d"
    prepared = Q.prepare(model, Q.get_minmax_qconfig())
    for _ in range(3):
        prepared(gpu.tensor(rng.standard_normal((2, 4, 5, 6, 6)).astype(np.float32), device="gpu"))
    q = Q.convert(prepared)
    assert isinstance(q[1], nnq.ConvReLU3d)
    x = gpu.tensor(rng.standard_normal((2, 4, 5, 6, 6)).astype(np.float32), device="gpu")
    h = q[0](x)
    y = q[1](h)
    hq = h.quant_source
    c = hq.codes.numpy().astype(np.int64) + (128 if hq.code_type == __import__("lucid_amd")._C.U8S8 else 0)
    zx = int(hq.zero_point.numpy())
    acc = conv_nd_direct(c - zx, q[1].weight_int8.numpy().astype(np.int64), (1, 1, 1), [(1, 1)] * 3, (1, 1, 1), 1)
    want = _expected_codes(acc, np.float32(hq.scale.numpy()), q[1], None, True)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)
