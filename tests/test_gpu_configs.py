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


@pytest.mark.parametrize("shape,geom,offset", [
    ((4, 64, 112, 112), ((3, 3), (2, 2), (1, 1)), 0),   # the ResNet-18 stem pool: one plane per workgroup
    ((3, 7, 33, 29), ((2, 3), (2, 1), (1, 1)), 0),      # odd planes: several per workgroup, unaligned starts
    ((3, 7, 33, 29), ((3, 3), (1, 1), (1, 1)), 1),      # x not 16-byte aligned: byte loads
    ((2, 3, 181, 181), ((3, 3), (2, 2), (1, 1)), 0),    # planes over the LDS budget: per-output kernel
])
def test_max_pool_codes_paths(gpu, shape, geom, offset):
    # max pooling of int8 codes through the C ABI on both kernels (plane-staged and per
    # output), against the oracle's pooling of the same values
    from lucid_amd import _C

    k, s, p = geom
    rng = np.random.default_rng(sum(shape) + offset)
    codes = rng.integers(-128, 128, shape, dtype=np.int64).astype(np.int8)
    N, C, H, W = shape
    OH, OW = (H + 2 * p[0] - k[0]) // s[0] + 1, (W + 2 * p[1] - k[1]) // s[1] + 1
    buf = gpu.tensor(np.concatenate([np.zeros(offset, np.int8), codes.ravel()]), device="gpu")
    y = gpu.empty((N, C, OH, OW), np.int8, "gpu")
    _C.call("lq_pool2d", _C.POOL_MAX, buf.data_ptr() + offset, _C.I8, None, None, N, C, H, W, OH, OW, k[0], k[1],
            s[0], s[1], p[0], p[1], 0, y.data_ptr(), None)
    gpu.synchronize()
    path = _C.last_path()
    assert path == ("pool per output" if H * W > 24576 else "pool planes"), path
    want = O.pool2d(codes.astype(np.float32), "max", k, s, p)
    np.testing.assert_array_equal(y.numpy().astype(np.float32), want)


# ------------------------------------------------------------------- config 5: ResNet-18


def _resnet18(nn, nnq, rng, num_classes=1000):
    from lucid_amd.bench_configs import resnet18

    return resnet18(rng, num_classes)


def _host(a):
    import lucid_amd as L

    return L.tensor(np.asarray(a, np.float32))


def _fuse_groups():
    from lucid_amd.bench_configs import resnet18_fuse_groups

    return resnet18_fuse_groups()


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


def test_resnet18_config5_network_vs_oracle(gpu, resnet_pipeline):
    # The whole converted network at batch 2 against the oracle's composition run end to end on
    # its own outputs (no device value feeds it): the input codes, the stem, the max pool and
    # every block's output codes bit for bit, the global average pool's float32 bits, then the
    # fc (a float weight-only product, within its scale-aware tolerance, so its codes may move
    # by one where a value sits on a rounding boundary) and the dequantized logits.
    from tests.test_gpu_conv import oracle_conv

    rng, _, q = resnet_pipeline
    x = rng.standard_normal((2, 3, 224, 224)).astype(np.float32)

    def grid(mod):
        return np.float32(mod.scale.numpy().reshape(-1)[0]), np.float32(mod.zero_point.numpy().reshape(-1)[0])

    def codes_of(t):
        assert t.is_code_backed
        return t.quant_source.codes.numpy()

    def conv(mod, c, s, z, relu, pad, stride):
        assert not mod.weight_zero_point.numpy().any()
        so, zo = grid(mod)
        out = oracle_conv(c, mod.weight_int8.numpy(), u8s8=True, za=float(z), stride=stride, pad=pad,
                          a_scale=s, w_scale=mod.weight_scale.numpy(),
                          bias=mod.bias.numpy() if mod.bias is not None else None, out_kind=O.OUT_QU8S8,
                          out_scale=float(so), out_zp=float(zo), qmin=0, qmax=255, relu=relu)
        return out, so, zo

    # device forward, module by module (the forward's own sequence)
    h = q.quant(_dev(gpu, x))
    dev = {"quant": codes_of(h)}
    h = q.conv1(h)
    dev["conv1"] = codes_of(h)
    h = q.maxpool(h)
    dev["maxpool"] = codes_of(h)
    blocks = [getattr(q, f"layer{i}")[j] for i in range(1, 5) for j in range(2)]
    for n, blk in enumerate(blocks):
        h = blk(h)
        dev[f"block{n}"] = codes_of(h)
    pooled_dev = q.avgpool(h)
    fc_dev = q.fc(q.flatten(pooled_dev))
    logits_dev = q.dequant(fc_dev).numpy()

    # the oracle's chain
    s0, z0 = grid(q.quant)
    c = O.quantize(x, O.recip_tensor(np.atleast_1d(s0))[0], z0, 0, 255, O.U8S8)
    np.testing.assert_array_equal(dev["quant"], c)
    c, s, z = conv(q.conv1, c, s0, z0, True, (3, 3, 3, 3), (2, 2))
    np.testing.assert_array_equal(dev["conv1"], c)
    c = O.pool2d(c.astype(np.float32), "max", kernel=(3, 3), stride=(2, 2), pad=(1, 1)).astype(np.int8)
    np.testing.assert_array_equal(dev["maxpool"], c)
    for n, blk in enumerate(blocks):
        st = tuple(blk.conv1.stride)
        a, sa, za = conv(blk.conv1, c, s, z, True, (1, 1, 1, 1), st)
        b, sb, zb = conv(blk.conv2, a, sa, za, False, (1, 1, 1, 1), (1, 1))
        if blk.downsample is not None:
            d, sd, zd = conv(blk.downsample[0], c, s, z, False, (0, 0, 0, 0), st)
        else:
            d, sd, zd = c, s, z
        t = (O.dequantize(b, O.U8S8, sb, zb) + O.dequantize(d, O.U8S8, sd, zd)).astype(np.float32)
        t = np.where(t <= 0, np.float32(0), t).astype(np.float32)
        s, z = grid(blk.skip)
        c = O.quantize(t, O.recip_tensor(np.atleast_1d(s))[0], z, 0, 255, O.U8S8)
        np.testing.assert_array_equal(dev[f"block{n}"], c, err_msg=f"block {n}")
    pooled = O.pool2d(O.dequantize(c, O.U8S8, s, z), "avg", adaptive=(1, 1))
    np.testing.assert_array_equal(pooled_dev.numpy().view(np.uint32), pooled.view(np.uint32))
    fc = q.fc
    assert not fc.weight_zero_point.numpy().any()
    y = O.gemv_w8(pooled.reshape(2, -1), fc.weight_int8.numpy(), fc.weight_scale.numpy(), None,
                  fc.bias.numpy() if fc.bias is not None else None)
    sf, zf = grid(fc)
    lo, hi = fc.out_qdtype.quant_min, fc.out_qdtype.quant_max
    ct = O.U8S8 if lo >= 0 else O.I8
    want = O.quantize(y.astype(np.float32), O.recip_tensor(np.atleast_1d(sf))[0], zf, lo, hi, ct)
    got = codes_of(fc_dev)
    diff = got.astype(np.int32) - want.astype(np.int32)
    print(f"fc codes off by one: {np.count_nonzero(diff)} of {diff.size}", flush=True)
    assert np.abs(diff).max() <= 1 and np.count_nonzero(diff) <= diff.size // 1000 + 1
    np.testing.assert_array_equal(logits_dev.view(np.uint32), O.dequantize(got, ct, sf, zf).view(np.uint32))


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

from lucid_amd.bench_configs import BATCH, D_MODEL, DECODE, FFN, HEADS, LAYERS, PREFILL, VOCAB  # noqa: E402


def _decoder(gpu, rng):
    from lucid_amd.bench_configs import decoder

    return decoder(rng)


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

    def __init__(self, gpu, dec, glue, batch, fp16_qkv=False):
        self.gpu, self.dec, self.glue, self.B = gpu, dec, glue, batch
        self.caches = [([], []) for _ in range(LAYERS)]
        self.fp16_qkv = fp16_qkv

    def step(self, tokens, pos0):
        """Feed ``tokens`` [B, n] at positions pos0 .. pos0 + n - 1; logits of the last one."""
        B, n = tokens.shape
        hd = D_MODEL // HEADS
        h = (self.glue["tok"][tokens] + self.glue["pos"][pos0:pos0 + n]).astype(np.float32)
        for li, layer in enumerate(self.dec.layers):
            qkv = _run_linear(self.gpu, layer.qkv, _ln(h).reshape(-1, D_MODEL)).reshape(B, n, 3, HEADS, hd)
            q, k, v = (qkv[:, :, i].transpose(0, 2, 1, 3) for i in range(3))
            if self.fp16_qkv:
                q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
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


# ----------------------------------------- config 4 on the device (the bench's runtime)


def test_dyn_linear_matches_module(gpu, decoder_pair):
    """The bench runtime's Linear (the module's four launches on caller buffers) equals
    nnqd.Linear.forward bit for bit, on the packed (M = 8) and row-major (M = 4096) paths."""
    from lucid_amd.bench_configs import DynLinear

    rng, _, qdec, _, _ = decoder_pair
    for name in ("qkv", "down"):
        mod = getattr(qdec.layers[1], name)
        dl = DynLinear(mod, BATCH * PREFILL)
        for M in (BATCH, BATCH * PREFILL):
            x = (rng.standard_normal((M, dl.K)) * 0.7).astype(np.float32)
            dx = _dev(gpu, x)
            y = gpu.empty((M, dl.N), np.float32, "gpu")
            dl(dx.data_ptr(), M, y.data_ptr(), None)
            np.testing.assert_array_equal(y.numpy().view(np.uint32), mod(dx).numpy().view(np.uint32),
                                          err_msg=f"{name} M={M}")


def test_int8_decoder_runtime(gpu, decoder_pair):
    """The device decoder (prefill 64 tokens, then 16 greedy steps replayed from one captured
    graph) against the host-glue runner fed the same fp16-rounded q / k / v: prefill and
    step logits close (cosine), the same greedy tokens almost everywhere; graph replay
    identical to eager execution."""
    import ctypes

    from lucid_amd import _C
    from lucid_amd.bench_configs import Graph, Int8Decoder

    _, _, qdec, glue, tokens = decoder_pair
    T, steps = 64, 16
    prompt = tokens[:, :T]
    rt = Int8Decoder(qdec, glue, batch=BATCH, max_prompt=T, max_positions=T + steps)
    st = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(st))
    rt.set_prompt(prompt)
    rt.prefill(st)
    _C.call("lq_stream_synchronize", st)
    logits0 = rt.logits.numpy().copy()
    eager = []
    for _ in range(4):
        rt.decode(st)
        _C.call("lq_stream_synchronize", st)
        eager.append(rt.next.numpy().copy())
    # the same from a captured decode step
    rt.prefill(st)
    g = Graph(rt.decode, st)
    toks, logits = [], []
    for _ in range(steps):
        g.launch()
        _C.call("lq_stream_synchronize", st)
        toks.append(rt.next.numpy().copy())
        logits.append(rt.logits.numpy().copy())
    _C.call("lq_stream_destroy", st)
    for a, b in zip(eager, toks):
        np.testing.assert_array_equal(a, b)
    # host reference, teacher-forced on the device's tokens
    r = _Runner(gpu, qdec, glue, BATCH, fp16_qkv=True)
    ref0 = r.step(prompt, 0)
    refs = []
    nxt = ref0.argmax(-1)
    feed = [logits0.argmax(-1)] + toks[:-1]
    for s in range(steps):
        refs.append(r.step(feed[s][:, None], T + s))

    def cos(a, b):
        a, b = a.astype(np.float64), b.astype(np.float64)
        return (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))

    assert cos(logits0, ref0).min() > 0.999, cos(logits0, ref0).min()
    assert min(cos(a, b).min() for a, b in zip(logits, refs)) > 0.995
    agree = np.mean([(t == rf.argmax(-1)).mean() for t, rf in zip(toks, refs)])
    assert agree > 0.9, agree
    assert (nxt == logits0.argmax(-1)).mean() > 0.9


def test_int8_decoder_one_launch_steps_bit_exact(gpu, decoder_pair):
    """Decode steps whose Linears run as one launch each (norm, input step and product in
    lq_dynamic_linear_packed_f32, the residual stream in two buffers) leave the same logits,
    tokens and KV cache, bit for bit, as the same steps through the separate launches."""
    import ctypes

    from lucid_amd import _C
    from lucid_amd.bench_configs import Int8Decoder

    _, _, qdec, glue, tokens = decoder_pair
    T, steps = 32, 6
    st = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(st))
    out = []
    for one in (False, True):
        rt = Int8Decoder(qdec, glue, batch=BATCH, max_prompt=T, max_positions=T + steps, one_launch=one)
        rt.set_prompt(tokens[:, :T])
        rt.prefill(st)
        rt.decode(st)  # the step's last product is the head's: its path note says which form ran
        assert ("dynamic linear one launch" in _C.last_path()) == one
        rt.prefill(st)
        logits = []
        for _ in range(steps):
            rt.decode(st)
            _C.call("lq_stream_synchronize", st)
            logits.append(rt.logits.numpy().copy())
        out.append((np.stack(logits), rt.next.numpy().copy(), rt.cache[-1][0].numpy().copy()))
    _C.call("lq_stream_destroy", st)
    for a, b in zip(out[0], out[1]):
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
