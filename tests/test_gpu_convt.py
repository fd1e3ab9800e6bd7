"""GPU parity of the transposed convolution (lq_stride_expand + the int8 / float convolution
kernels) against the oracle's direct scatter definition.

* nn.quantized.ConvTranspose2d over code-backed input: output codes bit-exact against the
  oracle's exact int64 scatter sums through the W8A8 epilogue;
* the float nn.ConvTranspose2d (and the quantized layer's literal path): against float64,
  within 1e-5 of sum |terms|;
* the flow of the reference's own test (lucid/test/unit/quantization/test_module_breadth.py:
  31-48): prepare with the default qconfig, calibrate, convert, mean relative error < 5%.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import assert_close_f32

pytestmark = pytest.mark.gpu

CASES = [  # (N, Cin, Cout, H, W, K, stride, pad, output_padding, dilation, groups)
    (2, 8, 4, 8, 8, 3, 2, 1, 1, 1, 1),
    (1, 16, 32, 5, 7, 4, 2, 1, 0, 1, 1),
    (2, 6, 4, 6, 5, 3, (1, 2), (0, 1), (0, 1), (2, 1), 2),
    (1, 64, 64, 7, 7, 3, 1, 1, 0, 1, 1),
    (1, 32, 16, 4, 4, 2, 3, 0, 2, 1, 1),
]


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


@pytest.mark.parametrize("case", CASES)
def test_quantized_conv_transpose_codes_exact(gpu, case):
    import lucid_amd.nn.quantized as nnq
    from lucid_amd._tensor import QuantSource, Tensor

    N, Cin, Cout, H, W, K, s, p, op, d, g = case
    s, p, op, d = _pair(s), _pair(p), _pair(op), _pair(d)
    rng = np.random.default_rng(Cin + Cout + H)
    m = nnq.ConvTranspose2d(Cin, Cout, K, s, p, op, d, g)
    w = rng.integers(-127, 128, (Cin, Cout // g, K, K)).astype(np.int8)
    ws = rng.uniform(1e-3, 1e-2, Cout // g).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    S, Z = np.float32(0.07), np.float32(120.0)
    m.weight_int8, m.weight_scale = gpu.tensor(w, device="gpu"), gpu.tensor(ws, device="gpu")
    m.weight_zero_point = gpu.tensor(np.zeros(Cout // g, np.float32), device="gpu")
    m.bias = gpu.tensor(b, device="gpu")
    m.scale, m.zero_point = gpu.tensor(S, device="gpu"), gpu.tensor(Z, device="gpu")
    xs, xz = np.float32(0.03), np.float32(131.0)
    codes = rng.integers(-128, 128, (N, Cin, H, W)).astype(np.int8)   # U8S8 form (c - 128)
    q = QuantSource(gpu.tensor(codes, device="gpu"), O.U8S8, gpu.tensor(xs, device="gpu"),
                    gpu.tensor(xz, device="gpu"), 0, 255)
    y = m(Tensor._code_backed(q, codes.shape))
    acc = O.conv_transpose2d_acc(codes, w, za=int(xz), x_u8s8=True, stride=s, pad=p, output_padding=op,
                                 dilation=d, groups=g)
    assert y.is_code_backed and y.shape == acc.shape
    Nn, _, OH, OW = acc.shape
    want = O.gemm_epilogue(acc.astype(np.int32).transpose(0, 2, 3, 1).reshape(-1, Cout), xs, np.tile(ws, g), b,
                           S, Z, 0, 255, O.OUT_QU8S8, False)
    want = want.reshape(Nn, OH, OW, Cout).transpose(0, 3, 1, 2)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)


@pytest.mark.parametrize("case", CASES[:3])
def test_float_conv_transpose_matches_float64(gpu, case):
    import lucid_amd.nn as nn

    N, Cin, Cout, H, W, K, s, p, op, d, g = case
    s, p, op, d = _pair(s), _pair(p), _pair(op), _pair(d)
    rng = np.random.default_rng(7 + Cin)
    m = nn.ConvTranspose2d(Cin, Cout, K, s, p, op, g, True, d).to("gpu")
    x = rng.standard_normal((N, Cin, H, W)).astype(np.float32)
    y = m(gpu.tensor(x, device="gpu")).numpy()
    w = m.weight.numpy().astype(np.float64)
    # the direct scatter definition in float64 (the oracle's integer routine is for codes)
    acc = _scatter_f64(x.astype(np.float64), w, s, p, op, d, g)
    ref = acc + m.bias.numpy().astype(np.float64)[None, :, None, None]
    assert_close_f32(y, ref)


def _scatter_f64(x, w, s, p, op, d, g):
    N, Cin, H, W = x.shape
    _, Cout_g, KH, KW = w.shape
    OH = (H - 1) * s[0] - 2 * p[0] + d[0] * (KH - 1) + op[0] + 1
    OW = (W - 1) * s[1] - 2 * p[1] + d[1] * (KW - 1) + op[1] + 1
    cg = Cin // g
    full = np.zeros((N, g * Cout_g, (H - 1) * s[0] + d[0] * (KH - 1) + 1 + op[0],
                     (W - 1) * s[1] + d[1] * (KW - 1) + 1 + op[1]))
    for gi in range(g):
        for kh in range(KH):
            for kw in range(KW):
                full[:, gi * Cout_g:(gi + 1) * Cout_g, kh * d[0]:kh * d[0] + (H - 1) * s[0] + 1:s[0],
                     kw * d[1]:kw * d[1] + (W - 1) * s[1] + 1:s[1]] += np.einsum(
                         "nchw,co->nohw", x[:, gi * cg:(gi + 1) * cg], w[gi * cg:(gi + 1) * cg, :, kh, kw])
    return full[:, :, p[0]:p[0] + OH, p[1]:p[1] + OW]


def test_conv_transpose_quantizes(gpu):
    # lucid/test/unit/quantization/test_module_breadth.py:31-48 (rank 2)
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.nn.layers import manual_seed

    Q = gpu.quantization
    manual_seed(2)
    rng = np.random.default_rng(2)
    m = nn.Sequential(nnq.QuantStub(), nn.ConvTranspose2d(8, 4, 3, stride=2, padding=1, output_padding=1),
                      nnq.DeQuantStub()).to("gpu")
    x = gpu.tensor(rng.standard_normal((2, 8, 8, 8)).astype(np.float32), device="gpu")
    yf = m(x).numpy()
    prepared = Q.prepare(m, Q.get_default_qconfig_mapping())
    for _ in range(6):
        prepared(gpu.tensor(rng.standard_normal((2, 8, 8, 8)).astype(np.float32), device="gpu"))
    qm = Q.convert(prepared)
    assert isinstance(qm[1], nnq.ConvTranspose2d)
    assert qm[1].weight_int8.dtype == np.int8 and qm[1].weight_scale.shape == (4,)
    yq = qm(x).numpy()
    assert yq.shape == yf.shape == (2, 4, 16, 16)
    assert np.abs(yf - yq).mean() / (np.abs(yf).mean() + 1e-9) < 0.05
    sd = qm.state_dict()
    assert "1.weight_int8" in sd and "1.scale" in sd and "1.zero_point" in sd
