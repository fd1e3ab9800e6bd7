"""Lucid's CPU composition of the model-level BASELINE configurations -- TEST AND BASELINE
INFRASTRUCTURE ONLY: ``bench.py``'s ``cpu_baseline`` leg times these, never the product.

Lucid's sidecar quantized modules compute in float32 on the CPU, one elementwise op per pass
(Accelerate there; numpy's OpenBLAS sgemm here): a static ``nnq.Linear`` / ``nnq.Conv2d``
dequantizes its int8 weight on every call, runs the float op and fake-quantizes the result
onto its activation grid (lucid/nn/quantized/linear.py:206-215, conv.py:126-134; the
convolution is im2col + sgemm, backend/cpu/methods/Conv.cpp:271-360); the dynamic
``nnqd.Linear`` first derives per-tensor affine uint8 qparams from the live input range and
fake-quantizes the input (dynamic/linear.py:85-92, _qparams.py:186-205).  The glue of the
decoder (layer norm, attention, GELU) is float32 numpy.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def fake_quantize(x: np.ndarray, s: float, z: float, qmin: int, qmax: int) -> np.ndarray:
    """(clip(rne(x * (1 / s)) + z, qmin, qmax) - z) * s, each step a float32 pass."""
    inv = F32(1.0) / F32(s)
    t = x * inv
    t = np.rint(t)
    t = t + F32(z)
    t = np.clip(t, F32(qmin), F32(qmax))
    t = t - F32(z)
    return t * F32(s)


def dequantize_rows(q: np.ndarray, s: np.ndarray, z: np.ndarray) -> np.ndarray:
    """Per-output-channel dequantize (axis 0): (float(q) - z) * s, two passes."""
    shape = (-1,) + (1,) * (q.ndim - 1)
    w = q.astype(F32)
    w = w - z.reshape(shape).astype(F32)
    return w * s.reshape(shape).astype(F32)


def affine_qparams(mn: float, mx: float, qmin: int = 0, qmax: int = 255) -> tuple[np.float32, np.float32]:
    """calculate_qparams per-tensor affine (range extended to 0, eps 1e-8)."""
    mn, mx = F32(min(mn, 0.0)), F32(max(mx, 0.0))
    s = max(F32((mx - mn) / F32(qmax - qmin)), F32(1e-8))
    z = np.clip(F32(qmin) - np.rint(mn / s), qmin, qmax)
    return F32(s), F32(z)


def dynamic_linear(x: np.ndarray, w: tuple) -> np.ndarray:
    """nnqd.Linear.forward: live-range qparams, fake-quantized input, dequantized weight,
    sgemm with the weight transposed, bias add."""
    q, s, z, b = w
    xs, xz = affine_qparams(float(x.min()), float(x.max()))
    xq = fake_quantize(x, xs, xz, 0, 255)
    y = xq @ dequantize_rows(q, s, z).T
    return y + b if b is not None else y


def random_weight(rng: np.random.Generator, n: int, k: int) -> tuple:
    """Symmetric per-channel int8 codes, scales and a bias of an n x k Linear (synthetic)."""
    q = rng.integers(-127, 128, (n, k), dtype=np.int64).astype(np.int8)
    return q, rng.uniform(1e-4, 1e-3, n).astype(F32), np.zeros(n, F32), rng.normal(0, 0.02, n).astype(F32)


# ------------------------------------------------------------------- configuration 3


def w8a8_linear(A: np.ndarray, B: np.ndarray, sa: np.ndarray, sb: np.ndarray, bias: np.ndarray,
                out_scale: float) -> np.ndarray:
    """The W8A8 Linear of the headline as Lucid's CPU path computes it (nn/quantized/
    linear.py:206-215): dequantize the int8 activations (per-row scale sa [M, 1], zero point 0)
    and weights (per-output-channel scale sb [N, 1]) in separate passes, fp32 sgemm with the
    weight transposed, bias add, then the multi-pass requantize onto the int8 output grid
    (multiply by the float32 reciprocal of out_scale, round half even, add zero point 0, clip,
    cast)."""
    xa = A.astype(F32)
    xa = xa - F32(0.0)
    xa = xa * sa
    wb = B.astype(F32)
    wb = wb - F32(0.0)
    wb = wb * sb
    y = xa @ wb.T
    y = y + bias
    t = y * (F32(1.0) / F32(out_scale))
    t = np.rint(t)
    t = t + F32(0.0)
    t = np.clip(t, -128, 127)
    return t.astype(np.int8)


# ------------------------------------------------------------------- configuration 1


def mlp_forward(x: np.ndarray, layers: list) -> np.ndarray:
    """Dynamic int8 MLP: Linear, ReLU (x <= 0 -> 0), Linear."""
    h = dynamic_linear(x, layers[0])
    h = np.where(h <= 0, F32(0), h).astype(F32)
    return dynamic_linear(h, layers[1])


# ------------------------------------------------------------------- configuration 4


def layer_norm(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    mu = x.mean(-1, keepdims=True, dtype=F32)
    c = x - mu
    var = (c * c).mean(-1, keepdims=True, dtype=F32)
    return c / np.sqrt(var + F32(eps))


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    return F32(0.5) * x * (F32(1) + np.tanh(F32(0.7978845608) * (x + F32(0.044715) * x * x * x)))


class Decoder:
    """Configuration 4 on the CPU: synthetic per-channel int8 weights of the decoder's shapes,
    a float32 KV cache, greedy steps."""

    def __init__(self, rng: np.random.Generator, layers=6, d=512, heads=8, ffn=2048, vocab=32000,
                 positions=640, batch=8) -> None:
        self.d, self.h, self.hd, self.B = d, heads, d // heads, batch
        self.layers = [tuple(random_weight(rng, n, k) for n, k in ((3 * d, d), (d, d), (ffn, d), (d, ffn)))
                       for _ in range(layers)]
        self.head = random_weight(rng, vocab, d)
        self.tok = rng.normal(0, 0.02, (vocab, d)).astype(F32)
        self.pos = rng.normal(0, 0.02, (positions, d)).astype(F32)
        self.k = [np.zeros((batch, heads, positions, self.hd), F32) for _ in range(layers)]
        self.v = [np.zeros((batch, heads, positions, self.hd), F32) for _ in range(layers)]

    def step(self, tokens: np.ndarray, pos0: int, trace: list | None = None) -> np.ndarray:
        """Feed tokens [B, n] at positions pos0 ..; returns the next greedy token of each row.

        ``trace``, when a list, receives one dict of intermediates per layer and a last one
        with the logits (the pins of this composition compare each stage on its own inputs)."""
        B, n = tokens.shape
        h = self.tok[tokens] + self.pos[pos0:pos0 + n]
        for li, (qkv_w, out_w, up_w, down_w) in enumerate(self.layers):
            rec = {"h_in": h}
            ln1 = layer_norm(h).reshape(B * n, self.d)
            qkv = dynamic_linear(ln1, qkv_w).reshape(B, n, 3, self.h, self.hd)
            q = qkv[:, :, 0].transpose(0, 2, 1, 3)
            self.k[li][:, :, pos0:pos0 + n] = qkv[:, :, 1].transpose(0, 2, 1, 3)
            self.v[li][:, :, pos0:pos0 + n] = qkv[:, :, 2].transpose(0, 2, 1, 3)
            K, V = self.k[li][:, :, :pos0 + n], self.v[li][:, :, :pos0 + n]
            att = (q @ K.transpose(0, 1, 3, 2)) * F32(1.0 / np.sqrt(self.hd))
            visible = np.arange(pos0 + n)[None, :] <= (pos0 + np.arange(n))[:, None]
            att = np.where(visible, att, F32(-np.inf))
            att = np.exp(att - att.max(-1, keepdims=True))
            att = att / att.sum(-1, keepdims=True)
            o = (att @ V).transpose(0, 2, 1, 3).reshape(B * n, self.d)
            proj = dynamic_linear(o, out_w).reshape(B, n, self.d)
            h = h + proj
            ln2 = layer_norm(h).reshape(B * n, self.d)
            up = dynamic_linear(ln2, up_w)
            f = gelu_tanh(up)
            down = dynamic_linear(f, down_w).reshape(B, n, self.d)
            if trace is not None:
                rec.update(ln1=ln1, qkv=qkv, K=K.copy(), V=V.copy(), o=o, proj=proj, h_mid=h, ln2=ln2,
                           up=up, f=f, down=down)
            h = h + down
            if trace is not None:
                rec["h_out"] = h
                trace.append(rec)
        lnf = layer_norm(h[:, -1])
        logits = dynamic_linear(lnf, self.head)
        if trace is not None:
            trace.append({"h": h, "lnf": lnf, "logits": logits})
        return logits.argmax(-1)


# ------------------------------------------------------------------- configuration 5


def conv_layer(x: np.ndarray, w: tuple, stride: int, pad: int, relu: bool, act: tuple,
               trace: dict | None = None) -> np.ndarray:
    """nnq.Conv2d(ReLU2d): dequantized weight, im2col + sgemm, bias, ReLU, fake-quantize onto
    the layer's uint8 activation grid.  x [N, C, H, W] float32 -> [N, Cout, OH, OW].
    ``trace``, when a dict, receives the float result before the fake-quantize."""
    q, s, z, b = w
    Cout, C, KH, KW = q.shape
    wd = dequantize_rows(q, s, z).reshape(Cout, -1)
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    cols = np.lib.stride_tricks.sliding_window_view(xp, (KH, KW), axis=(2, 3))[:, :, ::stride, ::stride]
    N, _, OH, OW = cols.shape[:4]
    cols = np.ascontiguousarray(cols.transpose(0, 2, 3, 1, 4, 5)).reshape(N * OH * OW, C * KH * KW)
    y = cols @ wd.T
    y = y + b
    if relu:
        y = np.where(y <= 0, F32(0), y).astype(F32)
    if trace is not None:
        trace["pre_quant"] = np.ascontiguousarray(y.reshape(N, OH, OW, Cout).transpose(0, 3, 1, 2))
    y = fake_quantize(y, act[0], act[1], 0, 255)
    return np.ascontiguousarray(y.reshape(N, OH, OW, Cout).transpose(0, 3, 1, 2))


RESNET18_CONVS = (  # (Cin, Cout, H_in, k, stride, pad) of all 20 convolutions, in order
    (3, 64, 224, 7, 2, 3),
    (64, 64, 56, 3, 1, 1), (64, 64, 56, 3, 1, 1), (64, 64, 56, 3, 1, 1), (64, 64, 56, 3, 1, 1),
    (64, 128, 56, 3, 2, 1), (128, 128, 28, 3, 1, 1), (64, 128, 56, 1, 2, 0), (128, 128, 28, 3, 1, 1),
    (128, 128, 28, 3, 1, 1),
    (128, 256, 28, 3, 2, 1), (256, 256, 14, 3, 1, 1), (128, 256, 28, 1, 2, 0), (256, 256, 14, 3, 1, 1),
    (256, 256, 14, 3, 1, 1),
    (256, 512, 14, 3, 2, 1), (512, 512, 7, 3, 1, 1), (256, 512, 14, 1, 2, 0), (512, 512, 7, 3, 1, 1),
    (512, 512, 7, 3, 1, 1),
)


def resnet18_conv_stack(rng: np.random.Generator, batch: int) -> list:
    """(input, weight, stride, pad) for every convolution of ResNet-18 at this batch: synthetic
    per-channel int8 weights and uint8-grid inputs of each layer's shape."""
    out = []
    for cin, cout, H, k, st, pd in RESNET18_CONVS:
        x = fake_quantize(rng.standard_normal((batch, cin, H, H)).astype(F32), 0.03, 128, 0, 255)
        q = rng.integers(-127, 128, (cout, cin, k, k), dtype=np.int64).astype(np.int8)
        w = (q, rng.uniform(1e-3, 1e-2, cout).astype(F32), np.zeros(cout, F32), rng.normal(0, 0.1, cout).astype(F32))
        out.append((x, w, st, pd))
    return out
