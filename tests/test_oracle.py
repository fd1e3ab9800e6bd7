"""Pins of the CPU oracle (no GPU): the reference's known-answer tests, PyTorch's
implementation of the same primitives (the independent oracle of Lucid's own parity
suite, committed as tests/golden/torch_quant.npz), closed forms and brute force.

Each check is chosen so a plausible slip in the oracle (dropped zero point, divide
instead of multiply-by-reciprocal, wrong rounding mode, transposed operand, wrong pack
order) fails at least one of them.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "torch_quant.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


# ------------------------------------------------------------ reference KATs
# lucid/test/unit/quantization/test_functional.py


def test_kat_round_trip_on_grid():
    x = np.array([-1.0, -0.3, 0.0, 0.7, 2.0], np.float32)
    q = O.quantize(x, O.recip_scalar(0.05), 0.0, -128, 127, O.I8)
    assert q.tolist() == [-20, -6, 0, 14, 40]
    dq = O.dequantize(q, O.I8, np.float32(0.05), 0.0)
    assert np.allclose(dq, x, atol=1e-6)


def test_kat_saturation():
    q = O.quantize(np.array([-1000.0, 1000.0], np.float32), O.recip_scalar(0.1), 0.0, -128, 127)
    assert q.tolist() == [-128, 127]


def test_kat_docstring_saturation():
    # _functional.py:161-163: 100.0 at s=0.05 saturates to 127, not 2000
    assert O.quantize(np.array([100.0], np.float32), O.recip_scalar(0.05), 0, -128, 127)[0] == 127


def test_kat_affine_zero_point():
    q = O.quantize(np.array([0.0], np.float32), O.recip_scalar(0.02), 128.0, 0, 255, O.I16)
    assert q.tolist() == [128]


def test_kat_fake_equals_dequant_of_quant():
    x = np.array([-1.0, -0.31, 0.0, 0.72, 2.0], np.float32)
    inv = O.recip_scalar(0.05)
    fq, _ = O.fake_quantize(x, inv, np.float32(0.05), 0.0, -128, 127)
    dq = O.dequantize(O.quantize(x, inv, 0.0, -128, 127), O.I8, np.float32(0.05), 0.0)
    assert np.array_equal(fq, dq)


def test_kat_ste_mask_per_tensor():
    x = np.array([-100.0, 0.2, 0.5, 100.0], np.float32)
    _, m = O.fake_quantize(x, O.recip_scalar(0.05), np.float32(0.05), 0.0, -128, 127)
    assert m.tolist() == [0.0, 1.0, 1.0, 0.0]


def test_kat_ste_mask_per_channel():
    w = np.array([[1.0, 2.0, 300.0], [-400.0, 0.5, 0.1]], np.float32)
    s = np.array([0.02, 0.03], np.float32)
    _, m = O.fake_quantize(w, O.recip_tensor(s), s, 0.0, -128, 127, ch_axis=0)
    assert m.tolist() == [[1.0, 1.0, 0.0], [0.0, 1.0, 1.0]]


def test_kat_per_channel_half_step():
    w = np.array([[1.0, 2.0, 3.0], [-4.0, 0.5, 0.1]], np.float32)
    s = np.array([0.03, 0.05], np.float32)
    q = O.quantize(w, O.recip_tensor(s), 0.0, -128, 127, ch_axis=0)
    dq = O.dequantize(q, O.I8, s, 0.0, ch_axis=0)
    bound = np.array([[0.03 / 2], [0.05 / 2]]) + 1e-6
    assert (np.abs(dq - w) <= bound).all()


def test_kat_qparams():
    s, z = O.calc_qparams(-1.0, 3.0, False, False, 0, 255)
    assert s.item() == pytest.approx(4.0 / 255.0, rel=1e-5) and 0 <= z.item() <= 255
    s, z = O.calc_qparams(-2.5, 2.0, True, True, -128, 127)
    assert z.item() == 0.0 and s.item() > 0
    s, _ = O.calc_qparams(0.0, 0.0, False, True, -128, 127)
    assert s.item() > 0
    # docstring examples, _qparams.py:165-177
    s, z = O.calc_qparams(-2.0, 6.0, False, False, 0, 255)
    assert round(s.item(), 4) == 0.0314 and int(z.item()) == 64
    s, z = O.calc_qparams(-0.8, 0.5, True, True, -128, 127)
    assert int(z.item()) == 0
    s, _ = O.calc_qparams(3.0, 3.0, False, True, -128, 127)
    assert s.item() > 0


def test_kat_symmetric_extremum_reciprocal_rounding():
    """test_functional.py:114-139: codes are round(x * (1/s)) with the float32 reciprocal;
    at each channel's extremum x/s is exactly 127.5, so a divide would round differently."""
    data = np.random.default_rng(0).standard_normal((64, 256)).astype(np.float32)
    mn, mx = O.minmax_per_channel(data, 1)
    scale, zp = O.calc_qparams(mn, mx, True, True, -128, 127)
    inv = np.float32(1.0) / scale
    codes = np.round(data * inv)
    expected_mask = ((codes >= -128) & (codes <= 127)).astype(np.float32)
    assert (expected_mask == 0.0).any()
    _, mask = O.fake_quantize(data, O.recip_tensor(scale), scale, zp, -128, 127, ch_axis=1)
    np.testing.assert_array_equal(mask, expected_mask)
    q = O.quantize(data, O.recip_tensor(scale), zp, -128, 127, ch_axis=1)
    np.testing.assert_array_equal(q, np.clip(codes, -128, 127))
    # dividing instead would differ at the extrema
    divided = np.clip(np.round(data / scale), -128, 127)
    assert (divided != q).any()


# lucid/test/unit/quantization/test_observer.py


def test_kat_observers():
    r = O.minmax(np.array([[-1.0, 2.0], [0.5, 3.0]], np.float32))
    r = O.minmax(np.array([[-2.0, 1.0]], np.float32), r)
    assert r.tolist() == [-2.0, 3.0]
    r = O.minmax(np.array([-1.0, 3.0], np.float32))
    s, z = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    assert s.item() == pytest.approx(4.0 / 255.0, rel=1e-5)
    r = O.minmax(np.array([-2.0, 2.0], np.float32), mode=O.OBS_EMA, c=0.5)
    r = O.minmax(np.array([-4.0, 4.0], np.float32), r, mode=O.OBS_EMA, c=0.5)
    assert r.tolist() == [-3.0, 3.0]
    mn, mx = O.minmax_per_channel(np.array([[1.0, 2.0, 3.0], [-4.0, 0.5, 0.1]], np.float32), 0)
    assert mn.tolist() == [1.0, -4.0] and mx.tolist() == [3.0, 0.5]
    _, z = O.calc_qparams(mn, mx, True, True, -128, 127)
    assert z.tolist() == [0.0, 0.0]
    # EMA docstring, observer.py:506-512: a spike moves the smoothed max by ~1%
    r = O.minmax(np.zeros(4, np.float32), mode=O.OBS_EMA, c=0.01)
    r = O.minmax(np.full(4, 1000.0, np.float32), r, mode=O.OBS_EMA, c=0.01)
    assert r[1] < 20.0


# -------------------------------------------------------- PyTorch fixtures


def test_torch_per_tensor_codes_fake_dequant(g):
    x = g["pt_x"]
    for i, (s, z, signed) in enumerate(zip(g["pt_scale"], g["pt_zp"], g["pt_signed"])):
        lo, hi = (-128, 127) if signed else (0, 255)
        inv = O.recip_scalar(float(s))
        np.testing.assert_array_equal(O.quantize(x, inv, z, lo, hi, O.I16), g["pt_codes"][i])
        fq, _ = O.fake_quantize(x, inv, np.float32(s), z, lo, hi)
        np.testing.assert_array_equal(fq, g["pt_fake"][i])
        dq = O.dequantize(g["pt_codes"][i], O.I16, np.float32(s), z)
        np.testing.assert_array_equal(dq, g["pt_dequant"][i])


def test_torch_per_channel(g):
    for ax in (0, 1):
        sc = g[f"pc{ax}_scale"]
        q = O.quantize(g["pc_w"], O.recip_tensor(sc), 0.0, -128, 127, O.I8, ch_axis=ax)
        np.testing.assert_array_equal(q, g[f"pc{ax}_codes"])
        fq, _ = O.fake_quantize(g["pc_w"], O.recip_tensor(sc), sc, 0.0, -128, 127, ch_axis=ax)
        np.testing.assert_array_equal(fq, g[f"pc{ax}_fake"])


def test_torch_observers(g):
    """Observer parity tolerances of lucid/test/parity/quantization/test_observer_parity.py."""
    r = np.array([np.inf, -np.inf], np.float32)
    e = r.copy()
    for b in g["obs_batches"]:
        r = O.minmax(b, r)
        e = O.minmax(b, e, mode=O.OBS_EMA, c=0.1)
    np.testing.assert_array_equal(r, g["obs_minmax_range"])
    s, z = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    assert s.item() == pytest.approx(float(g["obs_minmax_scale"][0]), abs=1e-6)
    assert abs(z.item() - float(g["obs_minmax_zp"][0])) <= 1
    s, _ = O.calc_qparams(e[0], e[1], False, False, 0, 255)
    assert s.item() == pytest.approx(float(g["obs_ema_scale"][0]), abs=1e-6)
    mn, mx = O.minmax_per_channel(g["obs_pc_x"], 0)
    s, _ = O.calc_qparams(mn, mx, True, True, -128, 127)
    np.testing.assert_allclose(s, g["obs_pc_scale"], atol=1e-6)


# ---------------------------------------------------- closed forms, invariants


def test_minmax_matches_numpy_and_propagates_nan():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(10007).astype(np.float32)
    assert O.minmax(x).tolist() == [x.min(), x.max()]
    x[777] = np.nan
    assert np.isnan(O.minmax(x)).all()
    assert np.isnan(O.minmax(np.array([1.0], np.float32), (np.nan, 2.0))[0])


def test_minmax_signed_zero_order():
    r = O.minmax(np.array([0.0, -0.0], np.float32))
    assert np.signbit(r[0]) and not np.signbit(r[1])
    r = O.minmax(np.array([-0.0, 0.0], np.float32))
    assert np.signbit(r[0]) and not np.signbit(r[1])


def test_minmax_per_channel_matches_numpy_any_axis():
    x = np.random.default_rng(2).standard_normal((5, 7, 9)).astype(np.float32)
    for ax in range(3):
        mn, mx = O.minmax_per_channel(x, ax)
        axes = tuple(a for a in range(3) if a != ax)
        np.testing.assert_array_equal(mn, x.min(axis=axes))
        np.testing.assert_array_equal(mx, x.max(axis=axes))


def test_quantize_nan_inf_edge_cases():
    x = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0], np.float32)
    q = O.quantize(x, O.recip_scalar(0.1), 5.0, -128, 127)
    assert q.tolist() == [0, 127, -128, 5, 5]  # NaN passes clip, then casts to 0
    q = O.quantize(x, O.recip_scalar(0.1), 0.0, 0, 255, O.I16)
    assert q.tolist() == [0, 255, 0, 0, 0]


def test_round_half_even():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5], np.float32)
    q = O.quantize(x, 1.0, 0.0, -128, 127)
    assert q.tolist() == [0, 2, 2, 0, -2, -2]


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 1000,
        rng.standard_normal(2000).astype(np.float32) * 1e-5,  # subnormal halves
        np.array([65504, 65519.99, 65520, 1e6, -1e6, np.inf, -np.inf, 0.0, -0.0,
                  2.0 ** -25, 2.0 ** -24 * 1.5, 6.1e-5, 1.0009765625 + 2 ** -12], np.float32),
    ])
    bits = O.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(bits, ref)


def test_gemm_acc_brute_force():
    rng = np.random.default_rng(4)
    for M, N, K in [(1, 1, 1), (3, 5, 7), (17, 33, 129), (64, 48, 256)]:
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        B = rng.integers(-128, 128, (N, K), dtype=np.int8)
        za, zb = int(rng.integers(-5, 6)), rng.integers(-3, 4, N)
        want = (A.astype(np.int64) - za) @ (B.astype(np.int64) - zb[:, None]).T
        np.testing.assert_array_equal(O.gemm_acc(A, B, za, zb), want)


def test_linear_reference_goldens():
    """F.linear against the reference's own checked-in goldens (the inputs regenerated by the
    recipe of lucid/test/numerical/golden/test_golden.py:55-70 and :31-40, the expected
    outputs read from the .npz files copied under tests/golden/), at that test's atol 1e-5.
    The square matmul golden catches a transposed operand (linear(a, b^T) == a @ b)."""
    here = os.path.dirname(__file__)
    rng = np.random.default_rng(0)
    x = rng.uniform(-1.0, 1.0, size=(2, 4)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, size=(3, 4)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, size=(3,)).astype(np.float32)
    want = np.load(os.path.join(here, "golden", "lucid_linear_2x4_4to3.npz"))["out"]
    np.testing.assert_allclose(O.linear(x, w, b), want, atol=1e-5, rtol=0)
    rng = np.random.default_rng(0)
    a = rng.uniform(-1.0, 1.0, size=(4, 4)).astype(np.float32)
    bm = rng.uniform(-1.0, 1.0, size=(4, 4)).astype(np.float32)
    want = np.load(os.path.join(here, "golden", "lucid_matmul_4x4.npz"))["out"]
    np.testing.assert_allclose(O.linear(a, bm.T), want, atol=1e-5, rtol=0)
    assert np.max(np.abs(O.linear(a, bm) - want)) > 1e-2  # the other orientation is far off


def test_linear_closed_forms():
    """Identity and permutation weights select input columns exactly; zero weights leave the
    bias; an empty K leaves the bias."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 7)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    np.testing.assert_array_equal(O.linear(x, np.eye(7, dtype=np.float32), b), x.astype(np.float64) + b)
    perm = rng.permutation(7)
    np.testing.assert_array_equal(O.linear(x, np.eye(7, dtype=np.float32)[perm]), x[:, perm])
    np.testing.assert_array_equal(O.linear(x, np.zeros((3, 7), np.float32), b[:3]),
                                  np.broadcast_to(b[:3].astype(np.float64), (5, 3)))
    np.testing.assert_array_equal(O.linear(np.zeros((2, 0), np.float32), np.zeros((4, 0), np.float32),
                                           b[:4]), np.broadcast_to(b[:4].astype(np.float64), (2, 4)))


def test_gemm_epilogue_structure():
    rng = np.random.default_rng(5)
    A = rng.integers(-127, 128, (8, 64), dtype=np.int8)
    B = rng.integers(-127, 128, (16, 64), dtype=np.int8)
    acc = O.gemm_acc(A, B)
    # unit scales, no bias: y is the accumulator converted exactly (|acc| < 2^24)
    y = O.gemm_w8a8(A, B, 1.0, 1.0)
    np.testing.assert_array_equal(y, acc.astype(np.float32))
    sa = rng.uniform(1e-3, 1e-1, 8).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-1, 16).astype(np.float32)
    bias = rng.standard_normal(16).astype(np.float32)
    y = O.gemm_w8a8(A, B, sa, sb, bias=bias)
    ref = acc.astype(np.float64) * sa[:, None] * sb[None, :] + bias
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)
    # requantized codes are the oracle quantize of the float output; FQ32 its dequantize
    for relu in (False, True):
        yf = O.gemm_w8a8(A, B, sa, sb, bias=bias, relu=relu)
        if relu:
            assert (yf >= 0).all()
        q = O.gemm_w8a8(A, B, sa, sb, bias=bias, out_scale=0.05, out_zp=3, qmin=-128, qmax=127,
                        out_kind=O.OUT_Q8, relu=relu)
        np.testing.assert_array_equal(q, O.quantize(yf, O.recip_tensor(np.float32(0.05)), 3.0,
                                                    -128, 127))
        fq = O.gemm_w8a8(A, B, sa, sb, bias=bias, out_scale=0.05, out_zp=3, qmin=-128,
                         qmax=127, out_kind=O.OUT_FQ32, relu=relu)
        np.testing.assert_array_equal(fq, O.dequantize(q, O.I8, np.float32(0.05), 3.0))
    h = O.gemm_w8a8(A, B, sa, sb, bias=bias, out_kind=O.OUT_F16)
    np.testing.assert_array_equal(h, O.gemm_w8a8(A, B, sa, sb, bias=bias).astype(np.float16))


def test_gemv_w8_vs_float64_dequantized():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 96)).astype(np.float32)
    W = rng.integers(-127, 128, (40, 96), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-1, 40).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    what = (W.astype(np.float32) * s[:, None]).astype(np.float32)
    want = x.astype(np.float64) @ what.T.astype(np.float64) + b
    np.testing.assert_allclose(O.gemv_w8(x, W, s, bias=b), want, rtol=1e-12, atol=1e-12)


def test_group_pack_closed_form():
    # one row, gs=16, bits=4: w = 0..15 gives min 0, s = 1, codes = w
    w = np.arange(16, dtype=np.float32)[None, :]
    packed, scales, biases = O.group_quantize(w, 16, 4)
    assert scales.tolist() == [[1.0]] and biases.tolist() == [[0.0]]
    want = [sum(int(c) << (4 * j) for j, c in enumerate(range(i * 8, i * 8 + 8))) for i in range(2)]
    assert packed.tolist() == [want]
    np.testing.assert_array_equal(O.group_dequantize(packed, scales, biases, 16, 4), w)
    # bits=8, gs=4: codes 0..255 spread, little end first
    w8 = np.array([[0.0, 255.0, 1.0, 128.0]], np.float32)
    p8, s8, b8 = O.group_quantize(w8, 4, 8)
    assert p8.tolist() == [[0 | (255 << 8) | (1 << 16) | (128 << 24)]]


def test_group_round_trip_half_step():
    rng = np.random.default_rng(7)
    w = rng.standard_normal((8, 256)).astype(np.float32)
    for bits in (4, 8):
        for gs in (32, 64, 128):
            p, s, b = O.group_quantize(w, gs, bits)
            wh = O.group_dequantize(p, s, b, gs, bits)
            step = np.repeat(s, gs, axis=1)
            assert (np.abs(wh - w) <= step / 2 + 1e-6).all()


def test_group_constant_group_exact():
    w = np.full((2, 64), 0.375, np.float32)
    p, s, b = O.group_quantize(w, 64, 4)
    np.testing.assert_array_equal(O.group_dequantize(p, s, b, 64, 4), w)


def test_bf16_round_ties_and_torch():
    """bfloat16 rounding: half-even ties at 1 (spacing 2^-7), the subnormal floor 2^-133,
    overflow past the largest finite value, signed zeros; and torch's float32 -> bfloat16
    conversion (round to nearest even) on values over the whole exponent range."""
    import torch

    ties = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8), 2.0 ** -134, 3 * 2.0 ** -134,
                     3.3961775e38, 3.4e38, -0.0])
    want = np.array([1.0, 1 + 2.0 ** -6, -1.0, 0.0, 2.0 ** -132, 3.3895314e38, np.inf, -0.0], np.float32)
    got = O.bf16_round(ties)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(200000) * np.exp(rng.uniform(-100, 87, 200000))).astype(np.float32)
    t = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(v).view(np.uint32), t.view(np.uint32))


def test_group_matmul_dtype_rule_closed_forms():
    """The dtype rule of quantized_matmul: one group of 64 codes equal to 1, x = e_0, scale
    1 + 2^-12 and group bias 2^-12 (neither a half value): in float32 the product is
    1 + 2^-12 + 2^-12; in half the scale rounds to 1 and the group bias stays 2^-12, so the
    float64 product 1 + 2^-12 rounds (half spacing 2^-10 at 1) to 1; a layer bias of 3 2^-11
    is cast to half (exact) and added in half: fl16(1 + 3 2^-11) = 1 + 2^-9.  bfloat16: the
    scale rounds to 1 (spacing 2^-7), the product to 1, and 1 + 3 2^-11 rounds to 1."""
    codes = np.ones((1, 64), np.uint32)
    packed = (codes.reshape(1, 8, 8) << (np.arange(8, dtype=np.uint32) * 4)).sum(-1).astype(np.uint32)
    np.testing.assert_array_equal(O.group_codes(packed, 4), np.ones((1, 64)))
    s = np.array([[1 + 2.0 ** -12]], np.float32)
    b = np.array([[2.0 ** -12]], np.float32)
    x = np.zeros((1, 64))
    x[0, 0] = 1.0
    assert O.group_matmul(x, packed, s, b, 64, 4)[0, 0] == np.float64(np.float32(1 + 2.0 ** -12)) + 2.0 ** -12
    assert O.group_matmul(x, packed, s, b, 64, 4, "f16")[0, 0] == 1.0
    lb = np.array([3 * 2.0 ** -11], np.float32)
    assert O.group_matmul(x, packed, s, b, 64, 4, "f16", bias=lb)[0, 0] == 1 + 2.0 ** -9
    assert O.group_matmul(x, packed, s, b, 64, 4, "bf16", bias=lb)[0, 0] == 1.0
    assert O.group_matmul(-x, packed, s, b, 64, 4, "f16", relu=True)[0, 0] == 0.0
    # float32 mode equals the float64 product against the pinned dequantize
    rng = np.random.default_rng(5)
    w = rng.standard_normal((12, 128)).astype(np.float32)
    for bits in (4, 8):
        p, sc, bi = O.group_quantize(w, 32, bits)
        xx = rng.standard_normal((3, 128))
        ref = xx @ O.group_dequantize(p, sc, bi, 32, bits).astype(np.float64).T
        np.testing.assert_allclose(O.group_matmul(xx, p, sc, bi, 32, bits), ref, rtol=1e-6, atol=1e-6)
        xt = rng.standard_normal((3, 12))
        np.testing.assert_allclose(O.group_matmul(xt, p, sc, bi, 32, bits, transpose=False),
                                   xt @ O.group_dequantize(p, sc, bi, 32, bits).astype(np.float64),
                                   rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------ convolution


def _im2col_conv_i64(xc, w, stride, dilation, groups):
    """Independent formulation: sliding windows (numpy) + int64 matmul per group."""
    from numpy.lib.stride_tricks import sliding_window_view

    N, C, H, W = xc.shape
    Cout, Cg, KH, KW = w.shape
    eh, ew = dilation[0] * (KH - 1) + 1, dilation[1] * (KW - 1) + 1
    win = sliding_window_view(xc, (eh, ew), axis=(2, 3))[:, :, ::stride[0], ::stride[1]]
    win = win[..., ::dilation[0], ::dilation[1]]  # [N, C, OH, OW, KH, KW]
    OH, OW = win.shape[2], win.shape[3]
    out = np.zeros((N, Cout, OH, OW), np.int64)
    Cog = Cout // groups
    for g in range(groups):
        cols = win[:, g * Cg:(g + 1) * Cg].transpose(0, 2, 3, 1, 4, 5).reshape(N * OH * OW, -1)
        wg = w[g * Cog:(g + 1) * Cog].reshape(Cog, -1).astype(np.int64)
        out[:, g * Cog:(g + 1) * Cog] = (cols.astype(np.int64) @ wg.T).reshape(N, OH, OW, Cog).transpose(0, 3, 1, 2)
    return out


def test_conv_acc_1x1_is_gemm(O):
    rng = np.random.default_rng(1)
    x = rng.integers(-128, 128, (2, 24, 5, 7)).astype(np.int8)
    w = rng.integers(-128, 128, (10, 24, 1, 1)).astype(np.int8)
    acc = O.conv2d_acc(x, w, za=-7)
    A = x.transpose(0, 2, 3, 1).reshape(-1, 24)
    want = O.gemm_acc(A, w.reshape(10, 24), za=-7)
    np.testing.assert_array_equal(acc.transpose(0, 2, 3, 1).reshape(-1, 10), want)


def test_conv_acc_delta_kernel_reproduces_input(O):
    rng = np.random.default_rng(2)
    x = rng.integers(-128, 128, (1, 3, 6, 5)).astype(np.int8)
    w = np.zeros((3, 3, 3, 3), np.int8)
    for c in range(3):
        w[c, c, 1, 1] = 1
    for u8s8, za in ((False, 5), (True, 131)):
        acc = O.conv2d_acc(x, w, za=za, x_u8s8=u8s8, pad=(1, 1, 1, 1))
        codes = x.astype(np.int64) + (128 if u8s8 else 0)
        np.testing.assert_array_equal(acc, codes - za)


@pytest.mark.parametrize("stride,dilation,groups", [((1, 1), (1, 1), 1), ((2, 1), (1, 2), 1),
                                                    ((2, 2), (2, 2), 2), ((1, 3), (1, 1), 4)])
def test_conv_acc_matches_windowed_matmul(O, stride, dilation, groups):
    rng = np.random.default_rng(sum(stride) + groups)
    x = rng.integers(-128, 128, (2, 8, 11, 13)).astype(np.int8)
    w = rng.integers(-128, 128, (8, 8 // groups, 3, 2)).astype(np.int8)
    acc = O.conv2d_acc(x, w, za=0, stride=stride, dilation=dilation, groups=groups)
    np.testing.assert_array_equal(acc, _im2col_conv_i64(x, w, stride, dilation, groups))


@pytest.mark.parametrize("mode,np_mode", [(1, "reflect"), (2, "edge"), (3, "wrap")])
def test_conv_padding_modes_match_numpy_pad(O, mode, np_mode):
    rng = np.random.default_rng(mode)
    x = rng.integers(-128, 128, (1, 4, 6, 7)).astype(np.int8)
    w = rng.integers(-128, 128, (5, 4, 3, 3)).astype(np.int8)
    pad = (2, 1, 1, 2)
    xp = np.pad(x, ((0, 0), (0, 0), (pad[0], pad[1]), (pad[2], pad[3])), mode=np_mode)
    want = O.conv2d_acc(xp, w, za=0)
    np.testing.assert_array_equal(O.conv2d_acc(x, w, za=0, pad=pad, mode=mode), want)
    xf = x.astype(np.float32) * 0.5
    np.testing.assert_array_equal(O.conv2d_f32(xf, w.astype(np.float32), pad=pad, mode=mode),
                                  O.conv2d_f32(xp.astype(np.float32) * 0.5, w.astype(np.float32)))


def test_conv_f32_against_float64(O):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 6, 9, 8)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = O.conv2d_f32(x, w, b, stride=(2, 1), pad=(1, 1, 0, 2), groups=2)
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (0, 2)))
    ref = np.zeros(y.shape)
    for g in range(2):
        for co in range(2 * g, 2 * g + 2):
            for oh in range(y.shape[2]):
                for ow in range(y.shape[3]):
                    patch = xp[:, 3 * g:3 * g + 3, 2 * oh:2 * oh + 3, ow:ow + 3]
                    ref[:, co, oh, ow] = (patch * w[co].astype(np.float64)).sum(axis=(1, 2, 3)) + b[co]
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------- histogram observer pins


def test_histc_closed_form():
    # bins of width 1 over [0, 8]: an interior value, a value on an inner edge (belongs to
    # the upper bin), the top edge (last bin), and values the reference skips.
    x = np.array([0.0, 0.5, 1.0, 3.25, 7.999, 8.0, -0.1, 8.1, np.nan, np.inf, -np.inf], np.float32)
    want = np.array([2, 1, 0, 1, 0, 0, 0, 2], np.float32)
    np.testing.assert_array_equal(O.histc(x, 8, 0.0, 8.0), want)


def test_hist_rebin_closed_forms():
    rng = np.random.default_rng(3)
    h = rng.integers(0, 50, 8).astype(np.float32)
    # twice as wide, same origin: target j collects sources 2j and 2j + 1
    np.testing.assert_array_equal(O.hist_rebin(h, 0.0, 8.0, 0.0, 16.0),
                                  np.concatenate([h[0::2] + h[1::2], np.zeros(4, np.float32)]))
    # twice as wide, centred: the old support lands on targets 4..7
    np.testing.assert_array_equal(O.hist_rebin(h, 0.0, 8.0, -8.0, 8.0),
                                  np.concatenate([np.zeros(4, np.float32), h[0::2] + h[1::2]]))
    # a point support (old_min == old_max) moves its whole mass to one bin
    r = O.hist_rebin(h, 2.0, 2.0, 0.0, 8.0)
    assert r[2] == h.sum() and np.count_nonzero(r) == 1
    # mass is conserved for any widening
    big = rng.integers(0, 1000, 2048).astype(np.float32)
    assert O.hist_rebin(big, -1.3, 2.7, -5.1, 9.4).sum() == big.sum()


def test_hist_clip_search_pins():
    # A flat histogram gains nothing from clipping: the full support (first to last centre).
    h = np.full(64, 10.0, np.float32)
    lo, hi = 0.0, 64.0
    assert O.hist_clip_search(h, lo, hi, 255) == (0.5, 63.5)
    # The reference's documented example (observer.py:785-798): one far outlier next to a
    # normal bulk is kept at 1e5 values and clipped at 1e6.
    rng = np.random.default_rng(0)
    for n, clipped in ((100_000, False), (1_000_000, True)):
        x = rng.standard_normal(n).astype(np.float32)
        x[0] = 50.0
        _, _, hist = O.histogram_observer([x], 2048)
        cmin, cmax = O.hist_clip_search(hist, float(x.min()), 50.0, 255)
        assert (cmax < 25.0) == clipped, (n, cmax)
    # The reference unit test (test_observer.py:64-76): a heavy tail makes the histogram
    # range no wider than min/max.
    data = np.concatenate([rng.standard_normal(3000), rng.uniform(5.0, 12.0, 150)]).astype(np.float32)
    mn, mx, hist = O.histogram_observer([data], 512)
    cmin, cmax = O.hist_clip_search(hist, mn, mx, 255)
    s_hist, _ = O.calc_qparams(np.float32(cmin), np.float32(cmax), False, False, 0, 255)
    s_mm, _ = O.calc_qparams(np.float32(mn), np.float32(mx), False, False, 0, 255)
    assert s_hist <= s_mm


# ------------------------------------------------------------------- activations


def _ulps(a, b):
    """Distance in float32 ulps (of the larger magnitude) between two arrays; differences
    below the smallest normal float32 count as 0 (a float32 exp overflows to inf where the
    exact result is subnormal, and the float32 composition then returns 0)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    u = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32)).astype(np.float64)
    d = np.abs(a - b)
    return np.where(d < np.finfo(np.float32).tiny, 0.0, d / u)


def test_activation_docstring_kats():
    # the examples of lucid/nn/functional/activations.py (printed to 4 decimals), and
    # hardswish's -0 at x = -4 (x * 0 keeps x's sign)
    f = np.float32
    x4 = np.array([-2.0, -1.0, 0.0, 1.0], f)
    np.testing.assert_array_equal(O.activation(x4, O.ACT_LEAKY_RELU, 0.1), f([-0.2, -0.1, 0.0, 1.0]))
    np.testing.assert_allclose(O.activation(x4, O.ACT_ELU, 1.0), [-0.8647, -0.6321, 0.0, 1.0], atol=5e-5)
    x5 = np.array([-4.0, -1.0, 0.0, 1.0, 4.0], f)
    hs = O.activation(x5, O.ACT_HARDSWISH)
    np.testing.assert_allclose(hs, [0.0, -0.3333, 0.0, 0.6667, 4.0], atol=5e-5)
    assert np.signbit(hs[0]) and not np.signbit(hs[2])
    np.testing.assert_allclose(O.activation(x5, O.ACT_HARDSIGMOID), [0.0, 0.3333, 0.5, 0.6667, 1.0], atol=5e-5)
    x3 = np.array([-2.0, 0.0, 2.0], f)
    np.testing.assert_allclose(O.activation(x3, O.ACT_SIGMOID), [0.1192, 0.5, 0.8808], atol=5e-5)
    np.testing.assert_allclose(O.activation(x3, O.ACT_TANH), [-0.964, 0.0, 0.964], atol=5e-4)


def test_activation_against_float64():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(20000) * 4, rng.uniform(-1e-3, 1e-3, 2000),
                        [-3.0, 3.0, -2.9999998, 2.9999998, 80.0, -80.0, -100.0, 100.0]]).astype(np.float32)
    xd = x.astype(np.float64)
    # sigmoid: three roundings around exp
    assert _ulps(O.activation(x, O.ACT_SIGMOID), 1.0 / (1.0 + np.exp(-xd))).max() <= 4
    assert _ulps(O.activation(x, O.ACT_TANH), np.tanh(xd)).max() <= 2
    # hardsigmoid: (x + 3) and / 6 each rounded once; the clamps are exact
    hsd = np.clip((xd + 3.0) / 6.0, 0.0, 1.0)
    assert _ulps(O.activation(x, O.ACT_HARDSIGMOID), hsd).max() <= 2
    assert _ulps(O.activation(x, O.ACT_HARDSWISH), xd * hsd).max() <= 3
    # elu: exp(x) - 1 cancels near 0, so the error there is absolute (about an ulp of 1)
    el = O.activation(x, O.ACT_ELU, 1.5)
    want = np.where(xd >= 0, xd, np.float64(np.float32(1.5)) * np.expm1(xd))
    assert np.all(np.abs(el - want) <= 4 * np.spacing(np.float32(1.5)) + 1e-7 * np.abs(want))
    # leaky_relu: one IEEE float32 multiply = the exact product rounded once
    lr = O.activation(x, O.ACT_LEAKY_RELU, 0.2)
    exact = np.where(xd >= 0, xd, np.float64(np.float32(0.2)) * xd).astype(np.float32)
    np.testing.assert_array_equal(lr, exact)


def test_activation_special_values():
    f = np.float32
    x = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0], f)
    for op in range(6):
        y = O.activation(x, op, 0.5)
        assert np.isnan(y[0]), op   # NaN passes every activation
    np.testing.assert_array_equal(O.activation(x[1:3], O.ACT_SIGMOID), f([1.0, 0.0]))
    np.testing.assert_array_equal(O.activation(x[1:3], O.ACT_TANH), f([1.0, -1.0]))
    np.testing.assert_array_equal(O.activation(x[1:3], O.ACT_HARDSIGMOID), f([1.0, 0.0]))
    np.testing.assert_array_equal(O.activation(x[1:3], O.ACT_ELU, 2.0), f([np.inf, -2.0]))
    # -0 >= 0 holds: leaky_relu and elu keep -0
    assert np.signbit(O.activation(x[3:4], O.ACT_LEAKY_RELU, 0.1)[0])
    assert np.signbit(O.activation(x[3:4], O.ACT_ELU, 1.0)[0])


# ---------------------------------------------------------------- table lookups


def test_embedding_bag_closed_forms():
    # integer-valued tables: every float32 sum below is exact, so sum / mean / max are the
    # textbook reductions over each bag's non-padding rows
    rng = np.random.default_rng(5)
    table = rng.integers(-50, 50, (30, 7)).astype(np.float32)
    idx = rng.integers(0, 30, 40)
    offsets = np.array([0, 0, 3, 10, 10, 25, 39])
    pad = int(idx[4])
    for mode in (O.BAG_SUM, O.BAG_MEAN, O.BAG_MAX):
        got = O.embedding_bag(table, idx, offsets, mode, padding_idx=pad)
        ends = list(offsets[1:]) + [idx.size]
        for b, (s, e) in enumerate(zip(offsets, ends)):
            keep = [int(r) for r in idx[s:e] if r != pad]
            if not keep:
                np.testing.assert_array_equal(got[b], 0.0)
                continue
            rows = table[keep].astype(np.float64)
            want = {O.BAG_SUM: rows.sum(0), O.BAG_MEAN: rows.sum(0) / len(keep), O.BAG_MAX: rows.max(0)}[mode]
            np.testing.assert_array_equal(got[b], want.astype(np.float32))


def test_embedding_bag_in_order_float32_sum():
    # non-exact sums: the bag is the sequential float32 accumulation (np.cumsum in float32 adds
    # in order), not a pairwise or float64 one; include_last_offset drops the tail
    rng = np.random.default_rng(6)
    table = (rng.standard_normal((50, 9)) * 1e3).astype(np.float32)
    table[::7] *= 1e-4
    idx = rng.integers(0, 50, 60)
    offsets = np.array([0, 17, 17, 44, 55])
    got = O.embedding_bag(table, idx, offsets, O.BAG_SUM, include_last_offset=True)
    assert got.shape == (4, 9)
    for b in range(4):
        rows = table[idx[offsets[b]:offsets[b + 1]]]
        want = np.cumsum(rows, axis=0, dtype=np.float32)[-1] if len(rows) else np.zeros(9, np.float32)
        np.testing.assert_array_equal(got[b], want)
    # 2-D input: one bag per row; per_sample_weights: the float32 products summed in order
    w = rng.standard_normal(60).astype(np.float32)
    got2 = O.embedding_bag(table, idx.reshape(6, 10), None, O.BAG_SUM, bag_len=10, per_sample_weights=w)
    for b in range(6):
        prod = (table[idx[10 * b:10 * b + 10]] * w[10 * b:10 * b + 10, None]).astype(np.float32)
        np.testing.assert_array_equal(got2[b], np.cumsum(prod, axis=0, dtype=np.float32)[-1])


def test_div6_rewrite_is_exact_for_every_float():
    # the GPU hardsigmoid / hardswish divide by 6 as a reciprocal multiply plus one fma
    # residual correction (IEEE division where |t| < 2^-125 or not finite); exhaustive over
    # all 2^32 inputs against the IEEE quotient Lucid computes
    assert O.div6_mismatches() == 0


# ----------------------------------------------------------------------------- pooling


def test_pool2d_closed_forms():
    rng = np.random.default_rng(12)
    x = rng.integers(-50, 50, (2, 3, 8, 12)).astype(np.float32)
    # non-overlapping windows: numpy block reductions (integer values: exact sums)
    blocks = x.reshape(2, 3, 4, 2, 4, 3)
    np.testing.assert_array_equal(O.pool2d(x, "max", (2, 3), (2, 3)), blocks.max(axis=(3, 5)))
    np.testing.assert_array_equal(O.pool2d(x, "avg", (2, 3), (2, 3)),
                                  (blocks.astype(np.float64).sum(axis=(3, 5)) / 6).astype(np.float32))
    # adaptive to 1 x 1 is the plane mean; to the input size it is the identity
    np.testing.assert_array_equal(O.pool2d(x, "avg", adaptive=(1, 1))[..., 0, 0],
                                  (x.astype(np.float64).sum(axis=(2, 3)) / 96).astype(np.float32))
    np.testing.assert_array_equal(O.pool2d(x, "avg", adaptive=(8, 12)), x)
    # padding: max skips it, avg counts it (or not)
    ones = np.ones((1, 1, 3, 3), np.float32)
    np.testing.assert_array_equal(O.pool2d(-ones, "max", (3, 3), (1, 1), (1, 1)), -ones)
    corner = O.pool2d(ones, "avg", (3, 3), (1, 1), (1, 1))[0, 0, 0, 0]
    assert corner == np.float32(4 / 9)
    assert O.pool2d(ones, "avg", (3, 3), (1, 1), (1, 1), count_include_pad=False)[0, 0, 0, 0] == 1.0
    # adaptive cells of 5 -> 3: [0, 2), [1, 4), [3, 5)
    v = np.arange(5, dtype=np.float32).reshape(1, 1, 1, 5)
    np.testing.assert_array_equal(O.pool2d(v, "max", adaptive=(1, 3))[0, 0, 0], [1, 3, 4])
    # NaN propagates through max
    x[0, 0, 0, 1] = np.nan
    assert np.isnan(O.pool2d(x, "max", (2, 3), (2, 3))[0, 0, 0, 0])


# -------------------------------------------------------------------- recurrent layers


def _rnn_weights(rng, mode, I, H, L=1, D=1):
    G = {"LSTM": 4, "GRU": 3}.get(mode, 1)
    w = {}
    for layer in range(L):
        for d in range(D):
            sfx = f"_l{layer}" + ("_reverse" if d else "")
            fan = I if layer == 0 else D * H
            w[f"weight_ih{sfx}"] = rng.uniform(-0.5, 0.5, (G * H, fan))
            w[f"weight_hh{sfx}"] = rng.uniform(-0.5, 0.5, (G * H, H))
            w[f"bias_ih{sfx}"] = rng.uniform(-0.5, 0.5, G * H)
            w[f"bias_hh{sfx}"] = rng.uniform(-0.5, 0.5, G * H)
    return w


def test_rnn_cell_closed_forms():
    B, H = 3, 5
    h = np.linspace(-1, 1, B * H).reshape(B, H)
    c = np.linspace(2, -2, B * H).reshape(B, H)
    # zero gate products: LSTM gates i = f = o = 1/2, g = 0; GRU r = z = 1/2, n = 0
    hl, cl = O.rnn_cell("LSTM", np.zeros((B, 4 * H)), np.zeros((B, 4 * H)), h, c)
    np.testing.assert_allclose(cl, 0.5 * c)
    np.testing.assert_allclose(hl, 0.5 * np.tanh(0.5 * c))
    hg, _ = O.rnn_cell("GRU", np.zeros((B, 3 * H)), np.zeros((B, 3 * H)), h)
    np.testing.assert_allclose(hg, 0.5 * h)
    # saturated LSTM gates: i = f = o = 1, g = tanh(big) = 1 -> c' = c + 1, h' = tanh(c + 1)
    big = np.full((B, 4 * H), 40.0)
    hl, cl = O.rnn_cell("LSTM", big, np.zeros((B, 4 * H)), h, c)
    np.testing.assert_allclose(cl, c + 1.0)
    np.testing.assert_allclose(hl, np.tanh(c + 1.0))
    # GRU with z -> 1 keeps h; relu RNN clips
    gx = np.zeros((B, 3 * H))
    gx[:, H:2 * H] = 40.0
    np.testing.assert_allclose(O.rnn_cell("GRU", gx, np.zeros((B, 3 * H)), h)[0], h)
    np.testing.assert_array_equal(O.rnn_cell("RNN_RELU", -np.ones((B, H)), np.zeros((B, H)), h)[0], 0.0)


def test_rnn_forward_structure():
    rng = np.random.default_rng(8)
    T, B, I, H = 6, 3, 4, 5
    x = rng.standard_normal((T, B, I))
    for mode in ("LSTM", "GRU", "RNN_TANH"):
        w = _rnn_weights(rng, mode, I, H, L=2, D=2)
        out, h_n, c_n = O.rnn_forward(mode, x, w, num_layers=2, bidirectional=True)
        assert out.shape == (T, B, 2 * H) and h_n.shape == (4, B, H)
        # the reverse direction of layer 0 is a forward pass over the time-reversed input
        w_rev = {k.replace("_reverse", ""): v for k, v in w.items() if k.endswith("_l0_reverse")}
        o1, _, _ = O.rnn_forward(mode, x[::-1], w_rev)
        l0, _, _ = O.rnn_forward(mode, x, {k: v for k, v in w.items() if "_l0" in k}, bidirectional=True)
        np.testing.assert_allclose(l0[:, :, H:], o1[::-1])
        # the last forward step's output is h_n of that direction; the reverse ends at t = 0
        np.testing.assert_allclose(out[-1, :, :H], h_n[2])
        np.testing.assert_allclose(out[0, :, H:], h_n[3])
        # layer 2 consumes layer 1's output
        w2 = {k.replace("_l1", "_l0"): v for k, v in w.items() if "_l1" in k}
        o2, _, _ = O.rnn_forward(mode, l0, w2, bidirectional=True)
        np.testing.assert_allclose(o2, out)


def test_rnn_forward_projection_reduces_to_a_plain_lstm():
    """A projection W_hr = [I_P | 0] keeps the first P hidden units.  The projected LSTM (W_hh
    [4H, P], layer-2 W_ih over the D P projected outputs) then equals an unprojected one whose
    weights read only those units (zero columns elsewhere), restricted to them; c is the same
    full-width cell state.  A projection applied to c, to the wrong side of the product, or
    left out of the recurrent input fails it."""
    rng = np.random.default_rng(21)
    T, B, I, H, P, L, D = 5, 3, 4, 6, 2, 2, 2
    x = rng.standard_normal((T, B, I))
    sel = np.zeros((P, H))
    sel[:, :P] = np.eye(P)
    proj, plain = {}, {}
    for layer in range(L):
        for d in range(D):
            sfx = f"_l{layer}" + ("_reverse" if d else "")
            w_ih = rng.uniform(-0.5, 0.5, (4 * H, I if layer == 0 else D * P))
            w_hh = rng.uniform(-0.5, 0.5, (4 * H, P))
            proj[f"weight_ih{sfx}"], proj[f"weight_hh{sfx}"], proj[f"weight_hr{sfx}"] = w_ih, w_hh, sel
            wide_hh = np.zeros((4 * H, H))
            wide_hh[:, :P] = w_hh
            if layer == 0:
                wide_ih = w_ih
            else:
                wide_ih = np.zeros((4 * H, D * H))
                for dd in range(D):
                    wide_ih[:, dd * H:dd * H + P] = w_ih[:, dd * P:(dd + 1) * P]
            plain[f"weight_ih{sfx}"], plain[f"weight_hh{sfx}"] = wide_ih, wide_hh
            for k in ("bias_ih", "bias_hh"):
                proj[k + sfx] = plain[k + sfx] = rng.uniform(-0.5, 0.5, 4 * H)
    h0 = rng.standard_normal((L * D, B, P)) * 0.5
    h0w = np.zeros((L * D, B, H))
    h0w[:, :, :P] = h0
    c0 = rng.standard_normal((L * D, B, H)) * 0.5
    out, h_n, c_n = O.rnn_forward("LSTM", x, proj, L, True, h0, c0)
    ow, hw, cw = O.rnn_forward("LSTM", x, plain, L, True, h0w, c0)
    assert out.shape == (T, B, D * P) and h_n.shape == (L * D, B, P) and c_n.shape == (L * D, B, H)
    for dd in range(D):
        np.testing.assert_allclose(out[:, :, dd * P:(dd + 1) * P], ow[:, :, dd * H:dd * H + P], atol=1e-12)
    np.testing.assert_allclose(h_n, hw[:, :, :P], atol=1e-12)
    np.testing.assert_allclose(c_n, cw, atol=1e-12)
    # a general projection is not the selector: the emitted state really is h_raw W_hr^T
    one = {k: v for k, v in proj.items() if k.endswith("_l0")}
    one["weight_hr_l0"] = rng.uniform(-1, 1, (P, H))
    o1, h1, c1 = O.rnn_forward("LSTM", x[:1], one)
    g = x[0] @ one["weight_ih_l0"].T + one["bias_ih_l0"] + one["bias_hh_l0"]
    s = 1.0 / (1.0 + np.exp(-g))
    c_ = s[:, :H] * np.tanh(g[:, 2 * H:3 * H])
    np.testing.assert_allclose(c1[0], c_, atol=1e-12)
    np.testing.assert_allclose(o1[0], (s[:, 3 * H:] * np.tanh(c_)) @ one["weight_hr_l0"].T, atol=1e-12)


# ------------------------------------------------------------ transposed convolution


@pytest.mark.parametrize("stride,pad,opad,dil,groups", [((2, 2), (1, 1), (1, 1), (1, 1), 1),
                                                        ((1, 2), (0, 1), (0, 1), (2, 1), 2),
                                                        ((3, 3), (2, 0), (2, 1), (1, 1), 1)])
def test_conv_transpose_is_the_adjoint_of_conv(stride, pad, opad, dil, groups):
    # <conv(a, W), b> = <a, conv_transpose(b, W)> over integers: the transposed convolution is
    # the adjoint of the convolution with the same stride / padding / dilation
    rng = np.random.default_rng(sum(stride) + groups)
    Cin, Cout, K = 4, 6, 3
    a = rng.integers(-20, 20, (2, Cin, 11, 9)).astype(np.int8)
    W = rng.integers(-20, 20, (Cout, Cin // groups, K, K)).astype(np.int8)
    y = O.conv2d_acc(a, W, stride=stride, pad=(pad[0], pad[0], pad[1], pad[1]), dilation=dil, groups=groups)
    b = rng.integers(-20, 20, y.shape).astype(np.int8)
    # conv weight [Cout, Cin_g, K, K] is the transposed-conv weight [Cout, Cin_g] with roles swapped:
    # as a transposed conv from Cout channels back to Cin, grouped the same way
    wt = W.reshape(groups, Cout // groups, Cin // groups, K, K).reshape(Cout, Cin // groups, K, K)
    back = O.conv_transpose2d_acc(b, wt, stride=stride, pad=pad, dilation=dil, groups=groups,
                                  output_padding=(a.shape[2] - ((y.shape[2] - 1) * stride[0] - 2 * pad[0]
                                                                + dil[0] * (K - 1) + 1),
                                                  a.shape[3] - ((y.shape[3] - 1) * stride[1] - 2 * pad[1]
                                                                + dil[1] * (K - 1) + 1)))
    assert back.shape == a.shape
    lhs = int((y.astype(np.int64) * b).sum())
    rhs = int((a.astype(np.int64) * back).sum())
    assert lhs == rhs


def test_conv_transpose_equals_conv_of_expanded_input():
    # the scatter definition against the stride-1 convolution of the stride-expanded input with
    # the flipped, channel-swapped kernel (the route the GPU layer takes), with a zero point
    rng = np.random.default_rng(3)
    N, Cin, Cout, H, W, K, s, p, op, d, g = 2, 6, 4, 5, 7, 3, 2, 1, 1, 1, 2
    x = rng.integers(-128, 128, (N, Cin, H, W)).astype(np.int8)
    w = rng.integers(-127, 128, (Cin, Cout // g, K, K)).astype(np.int8)
    za = 17
    want = O.conv_transpose2d_acc(x, w, za=za, stride=(s, s), pad=(p, p), output_padding=(op, op),
                                  dilation=(d, d), groups=g)
    xu = np.full((N, Cin, (H - 1) * s + 1, (W - 1) * s + 1), za, np.int8)
    xu[:, :, ::s, ::s] = x
    wc = w.reshape(g, Cin // g, Cout // g, K, K).transpose(0, 2, 1, 3, 4)[..., ::-1, ::-1].reshape(Cout, Cin // g, K, K)
    pt = d * (K - 1) - p
    got = O.conv2d_acc(xu, np.ascontiguousarray(wc), za=za, pad=(pt, pt + op, pt, pt + op), dilation=(d, d), groups=g)
    np.testing.assert_array_equal(got, want)


# ----------------------------------------------------- float glue of the int8 decoder


def test_glue_against_torch():
    """The decoder glue restatements against PyTorch's CPU implementations (the independent
    oracle of Lucid's parity suite) in float64: layer norm (with and without affine), the
    tanh GELU, and causal scaled-dot-product attention at a decode position."""
    import torch
    import torch.nn.functional as TF

    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 48)) * 3 + 1
    g, b = rng.standard_normal(48), rng.standard_normal(48)
    t = torch.from_numpy(x)
    np.testing.assert_allclose(O.layer_norm(x, eps=1e-5), TF.layer_norm(t, (48,), eps=1e-5).numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.layer_norm(x, g, b, 1e-5),
                               TF.layer_norm(t, (48,), torch.from_numpy(g), torch.from_numpy(b), 1e-5).numpy(),
                               rtol=1e-12, atol=1e-12)
    z = np.linspace(-8, 8, 101)
    np.testing.assert_allclose(O.gelu_tanh(z), TF.gelu(torch.from_numpy(z), approximate="tanh").numpy(),
                               rtol=1e-12, atol=1e-14)
    B, H, n, hd, pos0 = 2, 3, 4, 8, 5
    q = rng.standard_normal((B, H, n, hd)).astype(np.float16)
    k = rng.standard_normal((B, H, pos0 + n + 3, hd)).astype(np.float16)  # trailing keys unused
    v = rng.standard_normal((B, H, pos0 + n + 3, hd)).astype(np.float16)
    T = pos0 + n
    mask = torch.from_numpy(np.arange(T)[None, :] <= (pos0 + np.arange(n))[:, None])
    want = TF.scaled_dot_product_attention(torch.from_numpy(q.astype(np.float64)),
                                           torch.from_numpy(k[:, :, :T].astype(np.float64)),
                                           torch.from_numpy(v[:, :, :T].astype(np.float64)), attn_mask=mask,
                                           scale=0.125).numpy().transpose(0, 2, 1, 3)
    np.testing.assert_allclose(O.attention(q, k, v, pos0, 0.125), want, rtol=1e-12, atol=1e-12)


def test_glue_closed_forms():
    """A constant row normalizes to 0, two values to -1 / +1; gelu(x) - gelu(-x) = x;
    attention over one visible key returns that key's value, over identical keys the mean
    of the values; a later key never changes an earlier query."""
    np.testing.assert_array_equal(O.layer_norm(np.full((1, 7), 3.5)), np.zeros((1, 7)))
    np.testing.assert_allclose(O.layer_norm(np.array([[2.0, 6.0]]), eps=0.0), [[-1.0, 1.0]], rtol=1e-15)
    z = np.linspace(-5, 5, 41)
    np.testing.assert_allclose(O.gelu_tanh(z) - O.gelu_tanh(-z), z, atol=1e-12)
    rng = np.random.default_rng(9)
    v = rng.standard_normal((1, 1, 6, 4))
    q = rng.standard_normal((1, 1, 1, 4))
    k = rng.standard_normal((1, 1, 6, 4))
    np.testing.assert_allclose(O.attention(q, k, v, 0, 1.0)[0, 0, 0], v[0, 0, 0], rtol=1e-15)
    k_same = np.repeat(k[:, :, :1], 6, axis=2)
    np.testing.assert_allclose(O.attention(q, k_same, v, 5, 1.0)[0, 0, 0], v[0, 0].mean(0), rtol=1e-12)
    qq = rng.standard_normal((1, 1, 3, 4))
    a = O.attention(qq, k, v, 0, 0.5)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 2:] += 10
    v2[:, :, 2:] -= 3
    np.testing.assert_allclose(O.attention(qq, k2, v2, 0, 0.5)[:, :2], a[:, :2], rtol=1e-15)
