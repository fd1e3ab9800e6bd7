"""The model-level BASELINE configurations on the GPU, and the layers they add.

* pooling (lq_pool2d: max / average / adaptive over float32 or codes) against the oracle;
* config 5, a static-quantized ResNet-18 (3 x 224 x 224, batch 32, per-channel int8 weights,
  per-tensor uint8 activations calibrated on 16 random batches with MinMax observers, BN
  folded, requantize after each conv + BN + ReLU, residual adds on FloatFunctional): the
  prepare -> calibrate -> convert flow, one residual block bit-exact against the oracle's
  composition, and the quantized network against its float original;
* config 4, an int8-dynamic decoder (6 layers, d 512, 8 heads, FFN 2048, vocab 32000, batch
  8, prefill 512 then greedy decode): every Linear through quantize_dynamic, bit-exact against
  the oracle at the prefill (M = 4096) and decode (M = 8) shapes, and the quantized logits
  against the float decoder (attention and layer norm in float on the host, as the test's
  glue).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _dev(gpu, a):
    return gpu.tensor(np.ascontiguousarray(a), device="gpu")


# ----------------------------------------------------------------------------- pooling


@pytest.mark.parametrize("geom", [((3, 3), (2, 2), (1, 1)), ((2, 2), (2, 2), (0, 0)), ((3, 2), (1, 2), (1, 1))])
def test_pool_float_matches_oracle(gpu, geom):
    import lucid_amd.nn.functional as F

    k, s, p = geom
    rng = np.random.default_rng(sum(k) + sum(s))
    x = (rng.standard_normal((3, 5, 17, 14)) * 3).astype(np.float32)
    x[0, 0, 0, :3] = np.nan
    xd = _dev(gpu, x)
    got = F.max_pool2d(xd, k, s, p).numpy()
    want = O.pool2d(x, "max", k, s, p)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(np.nan_to_num(got), np.nan_to_num(want))
    for cip in (True, False):
        got = F.avg_pool2d(xd, k, s, p, count_include_pad=cip).numpy()
        want = O.pool2d(x, "avg", k, s, p, count_include_pad=cip)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
        np.testing.assert_array_equal(np.nan_to_num(got), np.nan_to_num(want))


@pytest.mark.parametrize("out", [(1, 1), (3, 5), (7, 7)])
def test_adaptive_avg_pool_matches_oracle(gpu, out):
    import lucid_amd.nn.functional as F

    rng = np.random.default_rng(out[0] * 10 + out[1])
    x = rng.standard_normal((2, 6, 9, 13)).astype(np.float32)
    np.testing.assert_array_equal(F.adaptive_avg_pool2d(_dev(gpu, x), out).numpy(),
                                  O.pool2d(x, "avg", adaptive=out))


def test_pool_over_codes(gpu):
    # a code-backed input: max pooling stays on the grid (bit-exact codes), average pooling
    # dequantizes then averages
    import lucid_amd.nn.functional as F
    from lucid_amd._tensor import QuantSource, Tensor

    rng = np.random.default_rng(21)
    x = (rng.standard_normal((2, 4, 12, 12)) * 2).astype(np.float32)
    s, z = np.float32(0.03), np.float32(111.0)
    codes = O.quantize(x, O.recip_tensor(np.array([s]))[0], z, 0, 255, O.U8S8)
    q = QuantSource(_dev(gpu, codes), O.U8S8, gpu.tensor(s, device="gpu"), gpu.tensor(z, device="gpu"), 0, 255)
    xq = Tensor._code_backed(q, x.shape)
    vals = O.dequantize(codes, O.U8S8, s, z)
    mp = F.max_pool2d(xq, 3, 2, 1)
    assert mp.is_code_backed
    np.testing.assert_array_equal(mp.numpy(), O.pool2d(vals, "max", (3, 3), (2, 2), (1, 1)))
    np.testing.assert_array_equal(F.adaptive_avg_pool2d(xq, 1).numpy(), O.pool2d(vals, "avg", adaptive=(1, 1)))


# ------------------------------------------------------------------- config 5: ResNet-18


def _resnet18(nn, nnq, rng, num_classes=1000):
    def bn(c):
        m = nn.BatchNorm2d(c)
        m.running_mean = _host(rng.normal(0, 0.1, c))
        m.running_var = _host(rng.uniform(0.5, 1.5, c))
        m.weight = nn.Parameter(_host(rng.normal(1, 0.1, c)))
        m.bias = nn.Parameter(_host(rng.normal(0, 0.1, c)))
        return m

    class BasicBlock(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.conv1 = nn.Conv2d(cin, cout, 3, stride=stride, padding=1, bias=False)
            self.bn1 = bn(cout)
            self.relu = nn.ReLU()
            self.conv2 = nn.Conv2d(cout, cout, 3, padding=1, bias=False)
            self.bn2 = bn(cout)
            self.downsample = (nn.Sequential(nn.Conv2d(cin, cout, 1, stride=stride, bias=False), bn(cout))
                               if stride != 1 or cin != cout else None)
            self.skip = nnq.FloatFunctional()

        def forward(self, x):
            out = self.relu(self.bn1(self.conv1(x)))
            out = self.bn2(self.conv2(out))
            identity = self.downsample(x) if self.downsample is not None else x
            return self.skip.add_relu(out, identity)

    class ResNet18(nn.Module):
        def __init__(self):
            super().__init__()
            self.quant = nnq.QuantStub()
            self.conv1 = nn.Conv2d(3, 64, 7, stride=2, padding=3, bias=False)
            self.bn1 = bn(64)
            self.relu = nn.ReLU()
            self.maxpool = nn.MaxPool2d(3, 2, 1)
            chans = [(64, 64, 1), (64, 128, 2), (128, 256, 2), (256, 512, 2)]
            for i, (cin, cout, st) in enumerate(chans, 1):
                setattr(self, f"layer{i}", nn.Sequential(BasicBlock(cin, cout, st), BasicBlock(cout, cout, 1)))
            self.avgpool = nn.AdaptiveAvgPool2d(1)
            self.flatten = nn.Flatten()
            self.fc = nn.Linear(512, num_classes)
            self.dequant = nnq.DeQuantStub()

        def forward(self, x):
            x = self.maxpool(self.relu(self.bn1(self.conv1(self.quant(x)))))
            for i in range(1, 5):
                x = getattr(self, f"layer{i}")(x)
            return self.dequant(self.fc(self.flatten(self.avgpool(x))))

    return ResNet18().eval()


def _host(a):
    import lucid_amd as L

    return L.tensor(np.asarray(a, np.float32))


def _fuse_groups():
    groups = [["conv1", "bn1", "relu"]]
    for i in range(1, 5):
        for b in range(2):
            p = f"layer{i}.{b}"
            groups += [[f"{p}.conv1", f"{p}.bn1", f"{p}.relu"], [f"{p}.conv2", f"{p}.bn2"]]
            if i > 1 and b == 0:
                groups.append([f"{p}.downsample.0", f"{p}.downsample.1"])
    return groups


@pytest.fixture(scope="module")
def reference_engine():
    """Configs 4 and 5 quantize Linears per channel (the int8 sidecar layers): pin the engine
    ("auto" would route group-divisible Linears to the group-wise QuantizedLinearMLX)."""
    import lucid_amd.backends as backends

    backends.quantized.engine = "reference"
    yield
    backends.quantized.engine = "auto"


@pytest.fixture(scope="module")
def resnet_pipeline(gpu, reference_engine):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.nn.layers import manual_seed

    Q = gpu.quantization
    manual_seed(5)
    rng = np.random.default_rng(5)
    model = _resnet18(nn, nnq, rng)
    fused = Q.fuse_modules(model, _fuse_groups()).to("gpu")
    prepared = Q.prepare(fused, Q.get_minmax_qconfig())
    for _ in range(16):   # 16 random calibration batches of the config
        prepared(_dev(gpu, rng.standard_normal((32, 3, 224, 224)).astype(np.float32)))
    fused_float = Q.fuse_modules(model, _fuse_groups()).to("gpu")   # the float original (BN folded)
    return rng, fused_float, Q.convert(prepared)


def test_resnet18_config5_converts(gpu, resnet_pipeline):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    _, _, q = resnet_pipeline
    assert isinstance(q.quant, nnq.Quantize) and isinstance(q.dequant, nnq.DeQuantize)
    assert isinstance(q.conv1, nnq.ConvReLU2d) and isinstance(q.bn1, nn.Identity)
    blk = q.layer2[0]
    assert isinstance(blk.conv1, nnq.ConvReLU2d) and isinstance(blk.conv2, nnq.Conv2d)
    assert isinstance(blk.downsample[0], nnq.Conv2d) and isinstance(blk.skip, nnq.QFunctional)
    assert isinstance(q.fc, nnq.Linear) and isinstance(q.maxpool, nn.MaxPool2d)
    assert q.layer1[0].conv1.weight_int8.dtype == np.int8
    assert q.quant.qdtype.quant_min == 0 and q.quant.qdtype.quant_max == 255   # uint8 activations


def test_resnet18_config5_block_exact(gpu, resnet_pipeline):
    # layer2's first block (stride 2, 1x1 downsample, residual add_relu) from the codes that
    # reach it: every output code equals the oracle's integer composition
    from tests.test_gpu_conv import oracle_conv

    rng, _, q = resnet_pipeline
    x = _dev(gpu, rng.standard_normal((2, 3, 224, 224)).astype(np.float32))
    h = q.layer1(q.maxpool(q.conv1(q.quant(x))))
    assert h.is_code_backed
    blk = q.layer2[0]
    y = blk(h)
    src = h.quant_source
    codes, s_in, z_in = src.codes.numpy(), src.scale.numpy(), src.zero_point.numpy()

    def conv(mod, c, s, z, relu, pad, stride):
        sw, zw = mod.weight_scale.numpy(), mod.weight_zero_point.numpy()
        assert not zw.any()
        out = oracle_conv(c, mod.weight_int8.numpy(), u8s8=True, za=float(z), stride=stride, pad=pad,
                          a_scale=s, w_scale=sw, bias=mod.bias.numpy() if mod.bias is not None else None,
                          out_kind=O.OUT_QU8S8, out_scale=float(mod.scale.numpy()),
                          out_zp=float(mod.zero_point.numpy()), qmin=0, qmax=255, relu=relu)
        return out, mod.scale.numpy(), mod.zero_point.numpy()

    a, sa, za = conv(blk.conv1, codes, s_in, z_in, True, (1, 1, 1, 1), (2, 2))
    b, sb, zb = conv(blk.conv2, a, sa, za, False, (1, 1, 1, 1), (1, 1))
    d, sd, zd = conv(blk.downsample[0], codes, s_in, z_in, False, (0, 0, 0, 0), (2, 2))
    t = (O.dequantize(b, O.U8S8, sb, zb) + O.dequantize(d, O.U8S8, sd, zd)).astype(np.float32)
    t = np.where(t <= 0, np.float32(0), t).astype(np.float32)
    S, Z = blk.skip.scale.numpy(), blk.skip.zero_point.numpy()
    want = O.quantize(t, O.recip_tensor(np.atleast_1d(S))[0], Z, 0, 255, O.U8S8)
    np.testing.assert_array_equal(y.quant_source.codes.numpy(), want)


def test_resnet18_config5_vs_float(gpu, resnet_pipeline):
    # the quantized network against its float original (BN folded) on a fresh batch of the
    # config's shape: a measured agreement, not a parity claim (int8 noise accumulates over
    # 20 layers of a random network)
    rng, fused_float, q = resnet_pipeline
    x = _dev(gpu, rng.standard_normal((32, 3, 224, 224)).astype(np.float32))
    yf = fused_float(x).numpy().astype(np.float64)
    yq = q(x).numpy().astype(np.float64)
    assert yq.shape == (32, 1000) and np.isfinite(yq).all()
    cos = (yf * yq).sum(1) / (np.linalg.norm(yf, axis=1) * np.linalg.norm(yq, axis=1))
    assert cos.min() > 0.9, cos.min()


# ------------------------------------------------------- config 4: int8-dynamic decoder

D_MODEL, HEADS, FFN, VOCAB, LAYERS = 512, 8, 2048, 32000, 6
BATCH, PREFILL, DECODE = 8, 512, 128


def _decoder(gpu, rng):
    """The decoder's Linears (random init, N(0, 0.02)) as a module tree quantize_dynamic can
    walk, plus the float glue parameters (embeddings, layer norms) kept on the host."""
    import lucid_amd.nn as nn

    def lin(k, n):
        m = nn.Linear(k, n)
        m.weight = nn.Parameter(_host(rng.normal(0, 0.02, (n, k))))
        m.bias = nn.Parameter(_host(rng.normal(0, 0.02, n)))
        return m

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv = lin(D_MODEL, 3 * D_MODEL)
            self.out = lin(D_MODEL, D_MODEL)
            self.up = lin(D_MODEL, FFN)
            self.down = lin(FFN, D_MODEL)

    class Decoder(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.Sequential(*[Layer() for _ in range(LAYERS)])
            self.head = lin(D_MODEL, VOCAB)

    glue = {"tok": rng.normal(0, 0.02, (VOCAB, D_MODEL)).astype(np.float32),
            "pos": rng.normal(0, 0.02, (PREFILL + DECODE, D_MODEL)).astype(np.float32)}
    return Decoder().to("gpu"), glue


def _ln(x):
    x = x.astype(np.float32)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return ((x - mu) / np.sqrt(var + 1e-5)).astype(np.float32)


def _gelu(x):
    return (0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))).astype(np.float32)


def _run_linear(gpu, mod, x2d):
    return mod(_dev(gpu, x2d)).numpy()


class _Runner:
    """One decoding session: causal attention over a KV cache and layer norm on the host in
    float32 (the test's glue), every Linear through ``dec`` on the GPU."""

    def __init__(self, gpu, dec, glue, batch):
        self.gpu, self.dec, self.glue, self.B = gpu, dec, glue, batch
        self.caches = [([], []) for _ in range(LAYERS)]

    def step(self, tokens, pos0):
        """Feed ``tokens`` [B, n] at positions pos0 .. pos0 + n - 1; logits of the last one."""
        B, n = tokens.shape
        hd = D_MODEL // HEADS
        h = (self.glue["tok"][tokens] + self.glue["pos"][pos0:pos0 + n]).astype(np.float32)
        for li, layer in enumerate(self.dec.layers):
            qkv = _run_linear(self.gpu, layer.qkv, _ln(h).reshape(-1, D_MODEL)).reshape(B, n, 3, HEADS, hd)
            q, k, v = (qkv[:, :, i].transpose(0, 2, 1, 3) for i in range(3))
            ks, vs = self.caches[li]
            ks.append(k)
            vs.append(v)
            K, V = np.concatenate(ks, 2), np.concatenate(vs, 2)
            att = (q @ K.transpose(0, 1, 3, 2)) / np.float32(np.sqrt(hd))
            qpos = pos0 + np.arange(n)[:, None]
            att = np.where(np.arange(K.shape[2])[None, :] <= qpos, att, -np.inf)
            att = np.exp(att - att.max(-1, keepdims=True))
            att = (att / att.sum(-1, keepdims=True)).astype(np.float32)
            o = (att @ V).transpose(0, 2, 1, 3).reshape(-1, D_MODEL)
            h = h + _run_linear(self.gpu, layer.out, o).reshape(B, n, D_MODEL)
            f = _gelu(_run_linear(self.gpu, layer.up, _ln(h).reshape(-1, D_MODEL)))
            h = h + _run_linear(self.gpu, layer.down, f).reshape(B, n, D_MODEL)
        return _run_linear(self.gpu, self.dec.head, _ln(h[:, -1])).astype(np.float32)


def _greedy(gpu, dec, glue, prompt, steps):
    """Prefill ``prompt`` [B, T], then ``steps`` greedy tokens: (prefill logits, tokens,
    logits of every step)."""
    r = _Runner(gpu, dec, glue, prompt.shape[0])
    T = prompt.shape[1]
    logits0 = r.step(prompt, 0)
    toks, logits, nxt = [], [], logits0.argmax(-1)
    for s in range(steps):
        toks.append(nxt)
        logits.append(r.step(nxt[:, None], T + s))
        nxt = logits[-1].argmax(-1)
    return logits0, np.stack(toks, 1), logits


def _forced(gpu, dec, glue, prompt, tokens):
    """The same session fed ``tokens`` [B, steps] instead of its own argmax (teacher forcing)."""
    r = _Runner(gpu, dec, glue, prompt.shape[0])
    T = prompt.shape[1]
    logits0 = r.step(prompt, 0)
    return logits0, [r.step(tokens[:, s:s + 1], T + s) for s in range(tokens.shape[1])]


@pytest.fixture(scope="module")
def decoder_pair(gpu, reference_engine):
    from lucid_amd.quantization import quantize_dynamic

    rng = np.random.default_rng(44)
    dec, glue = _decoder(gpu, rng)
    qdec = quantize_dynamic(dec)
    tokens = rng.integers(0, VOCAB, (BATCH, PREFILL))
    return rng, dec, qdec, glue, tokens


def test_decoder_config4_linears_exact(gpu, decoder_pair):
    # every distinct Linear shape at the decode (M = 8) and prefill (M = 4096) sizes,
    # bit-exact against the oracle's dynamic-quantization composition
    import lucid_amd.nn.quantized.dynamic as nnqd
    from tests.test_gpu_modules import _oracle_dynamic_linear

    rng, dec, qdec, _, _ = decoder_pair
    layer, qlayer = dec.layers[0], qdec.layers[0]
    assert all(isinstance(getattr(qlayer, n), nnqd.Linear) for n in ("qkv", "out", "up", "down"))
    assert isinstance(qdec.head, nnqd.Linear)
    cases = [("qkv", BATCH * PREFILL), ("down", BATCH * PREFILL), ("qkv", BATCH), ("out", BATCH), ("up", BATCH),
             ("down", BATCH)]
    for name, M in cases:
        f, q = getattr(layer, name), getattr(qlayer, name)
        K = f.weight.shape[1]
        x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
        want, _ = _oracle_dynamic_linear(x, f.weight.numpy(), f.bias.numpy())
        got = q(_dev(gpu, x)).numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"{name} M={M}")
    x = rng.standard_normal((BATCH, D_MODEL)).astype(np.float32)
    want, _ = _oracle_dynamic_linear(x, dec.head.weight.numpy(), dec.head.bias.numpy())
    np.testing.assert_array_equal(qdec.head(_dev(gpu, x)).numpy().view(np.uint32), want.view(np.uint32))


def test_decoder_config4_generation(gpu, decoder_pair):
    # prefill 512, then 128 greedy steps with the quantized Linears; the float decoder fed the
    # same tokens (teacher forcing) gives logits close to the quantized ones at every step (a
    # measured agreement of int8 dynamic quantization, not a parity claim)
    _, dec, qdec, glue, tokens = decoder_pair
    q0, qtok, qlogits = _greedy(gpu, qdec, glue, tokens, DECODE)
    assert qtok.shape == (BATCH, DECODE) and ((qtok >= 0) & (qtok < VOCAB)).all()
    f0, flogits = _forced(gpu, dec, glue, tokens, qtok)

    def cos(a, b):
        a, b = a.astype(np.float64), b.astype(np.float64)
        return (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))

    assert cos(q0, f0).min() > 0.99, cos(q0, f0).min()
    worst = min(cos(qs, fs).min() for qs, fs in zip(qlogits, flogits))
    assert worst > 0.98, worst
    agree = np.mean([(qs.argmax(-1) == fs.argmax(-1)).mean() for qs, fs in zip(qlogits, flogits)])
    assert agree > 0.8, agree
