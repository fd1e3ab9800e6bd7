"""Pins of the oracle's timed CPU composition (no GPU).

``bench.py``'s CPU column times ``oracle.lucid_minmax`` / ``lucid_quantize`` /
``lucid_dequantize`` (Lucid's one-op-per-pass elementwise path) and
``oracle/lucid_models.py`` (the dynamic MLP, the int8 decoder and the static conv layers
composed the way Lucid's sidecar modules compute them).  Each is checked here against the
pinned oracle functions of ``tests/test_oracle.py``:

* the multi-pass elementwise functions equal ``minmax`` / ``quantize`` / ``dequantize``
  bit for bit (2^20 elements with the configuration's x20 outliers, plus NaN / inf edges);
* the pieces of ``lucid_models`` (qparams, fake-quantize, weight dequantize, embedding sum)
  equal their pinned counterparts bit for bit;
* every float stage of the MLP, decoder and conv layers is compared, on the stage's own
  inputs (teacher forcing), with the pinned composition (``calc_qparams`` ->
  ``fake_quantize`` -> ``dequantize`` -> float64 ``linear`` / float32 ``conv2d_f32`` /
  float64 ``layer_norm`` / ``gelu_tanh`` / ``attention``) at the scale-aware rtol 1e-5;
* end to end, the requantized activation codes of the CPU composition and the pinned chain
  differ by at most one code, and the rate of such differences is reported and bounded.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
import oracle.lucid_models as LM
from _tolerance import assert_close_f32

F32 = np.float32


def _outlier_normal(rng: np.random.Generator, n: int) -> np.ndarray:
    x = rng.standard_normal(n).astype(F32)
    idx = rng.choice(n, n // 1000, replace=False)
    x[idx] *= F32(20.0)
    return x


# ------------------------------------------------ multi-pass elementwise functions


def test_lucid_elementwise_equals_pinned_at_2_20():
    rng = np.random.default_rng(20261202)
    n = 1 << 20
    x = _outlier_normal(rng, n)
    mn, mx = O.lucid_minmax(x)
    want = O.minmax(x, mode=O.OBS_REPLACE)
    assert np.float32(mn).tobytes() == want[0].tobytes() and np.float32(mx).tobytes() == want[1].tobytes()

    q = np.empty(n, np.int8)
    t0 = np.empty(n, F32)
    t1 = np.empty(n, F32)
    y = np.empty(n, F32)
    # symmetric qint8 (zero point 0) and an asymmetric qint8 grid with a nonzero zero point
    for symmetric, z in ((True, 0.0), (False, None)):
        s, zp = O.calc_qparams(np.float32(mn), np.float32(mx), symmetric, True, -128, 127)
        s, zp = F32(s), F32(zp if z is None else z)
        inv = O.recip_tensor(s)
        O.lucid_quantize(x, inv, zp, -128, 127, q, t0, t1)
        np.testing.assert_array_equal(q, O.quantize(x, inv, zp, -128, 127, O.I8))
        O.lucid_dequantize(q, s, zp, y, t0)
        np.testing.assert_array_equal(y.view(np.uint32), O.dequantize(q, O.I8, s, zp).view(np.uint32))


def test_lucid_elementwise_edges():
    x = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 2.5, -2.5, 0.5, 1.5, 1e30, -1e30, 127.5,
                  -128.5], F32)
    n = x.size
    q = np.empty(n, np.int8)
    t0, t1, y = np.empty(n, F32), np.empty(n, F32), np.empty(n, F32)
    for z in (0.0, 3.0, -7.0):
        O.lucid_quantize(x, F32(1.0), F32(z), -128, 127, q, t0, t1)
        np.testing.assert_array_equal(q, O.quantize(x, F32(1.0), F32(z), -128, 127, O.I8))
    O.lucid_dequantize(q, F32(0.05), F32(-7.0), y, t0)
    np.testing.assert_array_equal(y.view(np.uint32), O.dequantize(q, O.I8, F32(0.05), F32(-7.0)).view(np.uint32))
    mn, mx = O.lucid_minmax(x)  # NaN propagates
    assert np.isnan(mn) and np.isnan(mx)
    z2 = np.array([0.0, -0.0, 1.0, -1.0], F32)
    mn, mx = O.lucid_minmax(z2[[0, 1]])
    assert np.signbit(mn) and not np.signbit(mx)  # -0 < +0, whichever comes first
    mn, mx = O.lucid_minmax(z2[[1, 0]])
    assert np.signbit(mn) and not np.signbit(mx)


# ------------------------------------------------------------- lucid_models pieces


def _pinned_affine_qparams(x):
    r = O.minmax(x, mode=O.OBS_REPLACE)
    s, z = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    return F32(s), F32(z)


def _pinned_fake_quantize(x, s, z):
    y, _ = O.fake_quantize(x, O.recip_tensor(F32(s)), F32(s), F32(z), 0, 255)
    return y


def test_lucid_models_pieces_equal_pinned():
    rng = np.random.default_rng(7)
    for x in (_outlier_normal(rng, 64 * 784).reshape(64, 784),
              np.abs(rng.standard_normal((8, 33)).astype(F32)),        # range extended to 0
              -np.abs(rng.standard_normal((8, 33)).astype(F32)),
              np.zeros((3, 5), F32)):                                   # degenerate range -> eps
        s, z = LM.affine_qparams(float(x.min()), float(x.max()))
        ws, wz = _pinned_affine_qparams(x)
        assert s.tobytes() == ws.tobytes() and z.tobytes() == wz.tobytes()
        got = LM.fake_quantize(x, s, z, 0, 255)
        np.testing.assert_array_equal(got.view(np.uint32), _pinned_fake_quantize(x, s, z).view(np.uint32))
    # half-way points of the grid round to even codes in both
    s = F32(0.5)
    x = (np.arange(-40, 41, dtype=F32) * F32(0.25))
    np.testing.assert_array_equal(LM.fake_quantize(x, s, F32(3), 0, 255).view(np.uint32),
                                  _pinned_fake_quantize(x, s, F32(3)).view(np.uint32))
    q, sw, zw, _ = LM.random_weight(rng, 48, 40)
    np.testing.assert_array_equal(LM.dequantize_rows(q, sw, zw).view(np.uint32),
                                  O.dequantize(q, O.I8, sw, zw, ch_axis=0).view(np.uint32))
    q4 = rng.integers(-127, 128, (6, 3, 3, 3)).astype(np.int8)
    s4 = rng.uniform(1e-3, 1e-2, 6).astype(F32)
    np.testing.assert_array_equal(LM.dequantize_rows(q4, s4, np.zeros(6, F32)).view(np.uint32),
                                  O.dequantize(q4, O.I8, s4, np.zeros(6, F32), ch_axis=0).view(np.uint32))


def _pinned_dynamic_linear(x, w):
    """nnqd.Linear's forward from the pinned pieces: live per-tensor affine quint8 qparams,
    fake-quantized input, per-channel dequantized weight, float64 linear."""
    q, s, z, b = w
    xs, xz = _pinned_affine_qparams(x)
    xq = _pinned_fake_quantize(x, xs, xz)
    W = O.dequantize(q, O.I8, s, z, ch_axis=0)
    return O.linear(xq, W, b), (xs, xz)


def _code_diff(a, b, s, z):
    """Codes of two float tensors on one uint8 grid (the pinned quantize rule); returns the
    largest code difference and the fraction of elements that differ."""
    inv = O.recip_tensor(F32(s))
    ca = O.quantize(np.asarray(a, F32), inv, F32(z), 0, 255, O.I16).astype(np.int64)
    cb = O.quantize(np.asarray(b, F32), inv, F32(z), 0, 255, O.I16).astype(np.int64)
    d = np.abs(ca - cb)
    return int(d.max(initial=0)), float((d != 0).mean())


def test_dynamic_linear_matches_pinned_composition():
    rng = np.random.default_rng(11)
    x = _outlier_normal(rng, 64 * 784).reshape(64, 784)
    w = LM.random_weight(rng, 256, 784)
    want, _ = _pinned_dynamic_linear(x, w)
    assert_close_f32(LM.dynamic_linear(x, w), want)


def test_mlp_forward_matches_pinned_composition():
    """Configuration 1's shapes: Linear 784 -> 256, ReLU, Linear 256 -> 10, batch 64."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((64, 784)).astype(F32)
    layers = [LM.random_weight(rng, 256, 784), LM.random_weight(rng, 10, 256)]
    got = LM.mlp_forward(x, layers)
    # stage by stage on the CPU composition's own hidden activations
    h_cpu = LM.dynamic_linear(x, layers[0])
    h_cpu = np.where(h_cpu <= 0, F32(0), h_cpu).astype(F32)
    h_pin, _ = _pinned_dynamic_linear(x, layers[0])
    h_pin = np.where(h_pin <= 0, 0.0, h_pin)
    assert_close_f32(h_cpu, h_pin)
    want, _ = _pinned_dynamic_linear(h_cpu, layers[1])
    assert_close_f32(got, want)
    # end to end: the second layer's input codes of the two chains differ by <= 1 code
    s, z = _pinned_affine_qparams(h_cpu)
    worst, rate = _code_diff(h_cpu, h_pin.astype(F32), s, z)
    print(f"mlp hidden codes: worst {worst}, rate {rate:.2e}")
    assert worst <= 1 and rate < 5e-3


@pytest.fixture(scope="module")
def decoder_trace():
    rng = np.random.default_rng(13)
    dec = LM.Decoder(rng, layers=2, d=128, heads=4, ffn=256, vocab=1000, positions=16, batch=2)
    prompt = rng.integers(0, 1000, (2, 6))
    prefill: list = []
    nxt = dec.step(prompt, 0, trace=prefill)
    decode: list = []
    dec.step(nxt[:, None], 6, trace=decode)
    return dec, prompt, nxt, prefill, decode


@pytest.mark.parametrize("phase", ["prefill", "decode"])
def test_decoder_stages_match_pinned_composition(decoder_trace, phase):
    dec, prompt, nxt, prefill, decode = decoder_trace
    trace, tokens, pos0 = (prefill, prompt, 0) if phase == "prefill" else (decode, nxt[:, None], 6)
    B, n = tokens.shape
    np.testing.assert_array_equal(trace[0]["h_in"].view(np.uint32),
                                  O.embedding_sum(dec.tok, dec.pos, tokens, pos0).view(np.uint32))
    for li, rec in enumerate(trace[:-1]):
        qkv_w, out_w, up_w, down_w = dec.layers[li]
        assert_close_f32(rec["ln1"], O.layer_norm(rec["h_in"]).reshape(B * n, dec.d))
        want, _ = _pinned_dynamic_linear(rec["ln1"], qkv_w)
        assert_close_f32(rec["qkv"].reshape(B * n, -1), want)
        q = rec["qkv"][:, :, 0].transpose(0, 2, 1, 3)
        att = O.attention(q, rec["K"], rec["V"], pos0, 1.0 / np.sqrt(dec.hd))
        assert_close_f32(rec["o"], att.reshape(B * n, dec.d))
        want, _ = _pinned_dynamic_linear(rec["o"], out_w)
        assert_close_f32(rec["proj"].reshape(B * n, dec.d), want)
        np.testing.assert_array_equal(rec["h_mid"], rec["h_in"] + rec["proj"])
        assert_close_f32(rec["ln2"], O.layer_norm(rec["h_mid"]).reshape(B * n, dec.d))
        want, _ = _pinned_dynamic_linear(rec["ln2"], up_w)
        assert_close_f32(rec["up"], want)
        assert_close_f32(rec["f"], O.gelu_tanh(rec["up"]))
        want, _ = _pinned_dynamic_linear(rec["f"], down_w)
        assert_close_f32(rec["down"].reshape(B * n, dec.d), want)
        np.testing.assert_array_equal(rec["h_out"], rec["h_mid"] + rec["down"])
        if li + 1 < len(trace) - 1:
            np.testing.assert_array_equal(trace[li + 1]["h_in"], rec["h_out"])
        # the up projection's input codes: CPU layer norm vs float64 layer norm
        s, z = _pinned_affine_qparams(rec["ln2"])
        worst, rate = _code_diff(rec["ln2"], O.layer_norm(rec["h_mid"]).reshape(B * n, dec.d), s, z)
        print(f"{phase} layer {li} ln2 codes: worst {worst}, rate {rate:.2e}")
        assert worst <= 1 and rate < 5e-3
    last = trace[-1]
    assert_close_f32(last["lnf"], O.layer_norm(last["h"][:, -1]))
    want, _ = _pinned_dynamic_linear(last["lnf"], dec.head)
    assert_close_f32(last["logits"], want)


def test_conv_layer_matches_pinned_composition():
    """A ResNet-18 3x3 layer's composition at a reduced batch and size: float conv of the
    dequantized weight (stage compared with the pinned float conv), bias, ReLU, then the
    fake-quantize onto the layer's uint8 grid (bit-exact with the pinned rule)."""
    rng = np.random.default_rng(14)
    for cin, cout, H, k, st, pd in ((16, 24, 12, 3, 1, 1), (8, 16, 15, 3, 2, 1), (3, 8, 20, 7, 2, 3),
                                    (16, 32, 12, 1, 2, 0)):
        x = LM.fake_quantize(rng.standard_normal((2, cin, H, H)).astype(F32), 0.03, 128, 0, 255)
        q = rng.integers(-127, 128, (cout, cin, k, k)).astype(np.int8)
        w = (q, rng.uniform(1e-3, 1e-2, cout).astype(F32), np.zeros(cout, F32),
             rng.normal(0, 0.1, cout).astype(F32))
        act = (F32(0.02), F32(5.0))
        tr: dict = {}
        got = LM.conv_layer(x, w, st, pd, True, act, trace=tr)
        Wd = O.dequantize(q, O.I8, w[1], w[2], ch_axis=0)
        pin = O.conv2d_f32(x, Wd, w[3], (st, st), (pd, pd, pd, pd))
        pin = np.where(pin <= 0, F32(0), pin).astype(F32)
        assert_close_f32(tr["pre_quant"], pin)
        np.testing.assert_array_equal(got.view(np.uint32),
                                      _pinned_fake_quantize(tr["pre_quant"], *act).view(np.uint32))
        worst, rate = _code_diff(tr["pre_quant"], pin, *act)
        print(f"conv {cin}->{cout} k{k}/{st} codes: worst {worst}, rate {rate:.2e}")
        assert worst <= 1 and rate < 5e-3


def test_w8a8_linear_matches_pinned_integer_composition():
    """The headline's CPU step (dequantize A and B, fp32 sgemm, bias, multi-pass requantize)
    against the pinned integer composition (exact int32 sum, then the epilogue): its float
    result before the requantize within the scale-aware rtol 1e-5 of the float64 product, and
    the int8 codes within one code, at a reported rate."""
    rng = np.random.default_rng(15)
    M, N, K = 64, 96, 512
    A = rng.integers(-127, 128, (M, K)).astype(np.int8)
    B = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = rng.uniform(1e-3, 1e-1, (M, 1)).astype(F32)
    sb = rng.uniform(1e-3, 1e-1, (N, 1)).astype(F32)
    bias = rng.standard_normal(N).astype(F32)
    got = LM.w8a8_linear(A, B, sa, sb, bias, 64.0).astype(np.int64)
    acc = O.gemm_acc(A, B).astype(np.float64)
    y64 = acc * (sa.astype(np.float64) * sb.astype(np.float64).T) + bias
    want_codes = O.gemm_w8a8(A, B, sa.ravel(), sb.ravel(), bias=bias, out_scale=64.0, out_kind=O.OUT_Q8).astype(np.int64)
    d = np.abs(got - want_codes)
    print(f"w8a8 codes vs the integer composition: worst {d.max()}, rate {(d != 0).mean():.2e}")
    assert d.max() <= 1 and (d != 0).mean() < 5e-3
    # the float stage: the codes are the pinned rule applied to a float32 product close to y64
    float_codes = O.quantize(y64.astype(F32), O.recip_tensor(F32(64.0)), 0.0, -128, 127, O.I8).astype(np.int64)
    assert np.abs(got - float_codes).max() <= 1
