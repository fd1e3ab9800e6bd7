"""GPU parity of the int8 implicit-GEMM Conv2d (lq_conv2d_i8) and the float helpers.

* int8 conv: bit-exact against the oracle's brute-force int64 convolution followed by the
  oracle's W8A8 epilogue, for every output kind, strides, dilations, groups (incl.
  depthwise), padding modes, signed and unsigned activation grids, ragged channel counts
  and output sizes that are not multiples of 4 (the scalar store path);
* the packed weight layout and its code sums: against a numpy restatement;
* float conv (lq_conv2d_f32) and eval BatchNorm (lq_batch_norm_f32): bit-exact against the
  oracle's restatement in the same op order.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

_OUT_DT = {O.OUT_I32: np.int32, O.OUT_F32: np.float32, O.OUT_F16: np.float16, O.OUT_Q8: np.int8,
           O.OUT_QU8: np.uint8, O.OUT_FQ32: np.float32, O.OUT_Q16: np.int16, O.OUT_QU8S8: np.int8}
GRID = {O.OUT_Q8: (-128, 127), O.OUT_QU8: (0, 255), O.OUT_FQ32: (0, 255), O.OUT_Q16: (0, 255),
        O.OUT_QU8S8: (0, 255)}


def _dev(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


def pack_conv_weights(L, w):
    from lucid_amd import _C

    Cout, Cg, KH, KW = w.shape
    nbytes = _C.lib().lq_conv2d_weight_pack_size(Cout, Cg, KH, KW)
    wp = L.empty((nbytes,), np.int8, "gpu")
    sums = L.empty((Cout,), np.int32, "gpu")
    wd = _dev(L, w)  # held until the launch has been issued and finished
    _C.call("lq_conv2d_pack_weights_i8", wd.data_ptr(), Cout, Cg, KH, KW, wp.data_ptr(),
            sums.data_ptr(), None)
    _C.synchronize()
    return wp, sums


def run_conv(L, x, w, *, u8s8=False, za=None, stride=(1, 1), pad=(0, 0, 0, 0), dilation=(1, 1),
             groups=1, mode=0, a_scale=0.02, w_scale=None, bias=None, out_kind=O.OUT_QU8S8,
             out_scale=0.1, out_zp=128.0, qmin=0, qmax=255, relu=False):
    from lucid_amd import _C

    N, C, H, W = x.shape
    Cout, _, KH, KW = w.shape
    wp, sums = pack_conv_weights(L, w)
    OH, OW = O.conv_out_hw(H, W, KH, KW, stride, pad, dilation)
    y = L.empty((N, Cout, OH, OW), _OUT_DT[out_kind], "gpu")
    ws_bytes = _C.lib().lq_conv2d_i8_workspace_size(N, C, H, W, Cout, KH, KW, *stride, *pad, *dilation, groups)
    ws = L.empty((max(ws_bytes, 16),), np.int8, "gpu")
    keep = []

    def opt(v):
        if v is None:
            return None
        t = _dev(L, np.asarray(v, np.float32))
        keep.append(t)
        return t.data_ptr()

    if w_scale is None:
        w_scale = np.full(Cout, 0.01, np.float32)
    xd = _dev(L, x)  # device inputs stay referenced through the call (an inline temporary
    # would be freed, and its block reused by the next argument, before the launch)
    _C.call("lq_conv2d_i8", xd.data_ptr(), _C.U8S8 if u8s8 else _C.I8, N, C, H, W,
            wp.data_ptr(), sums.data_ptr(), Cout, KH, KW, stride[0], stride[1], *pad, dilation[0],
            dilation[1], groups, mode, opt(np.float32(a_scale)), opt(None if za is None else [za]),
            opt(w_scale), opt(bias), opt(np.float32(out_scale)), opt(np.float32(out_zp)), qmin, qmax,
            out_kind, _C.EPI_RELU if relu else 0, y.data_ptr(), ws.data_ptr(), ws_bytes, None)
    return y.numpy()


def oracle_conv(x, w, *, u8s8=False, za=None, stride=(1, 1), pad=(0, 0, 0, 0), dilation=(1, 1),
                groups=1, mode=0, a_scale=0.02, w_scale=None, bias=None, out_kind=O.OUT_QU8S8,
                out_scale=0.1, out_zp=128.0, qmin=0, qmax=255, relu=False):
    Cout = w.shape[0]
    if w_scale is None:
        w_scale = np.full(Cout, 0.01, np.float32)
    acc = O.conv2d_acc(x, w, za=0 if za is None else za, x_u8s8=u8s8, stride=stride, pad=pad,
                       dilation=dilation, groups=groups, mode=mode)
    N, _, OH, OW = acc.shape
    y = O.gemm_epilogue(acc.transpose(0, 2, 3, 1).reshape(-1, Cout), np.float32(a_scale), w_scale,
                        bias, out_scale, out_zp, qmin, qmax, out_kind, relu)
    return y.reshape(N, OH, OW, Cout).transpose(0, 3, 1, 2)


def _check(got, want, kind):
    if kind == O.OUT_F16:
        np.testing.assert_array_equal(got.view(np.uint16), np.ascontiguousarray(want).view(np.uint16))
    else:
        np.testing.assert_array_equal(got.view(np.uint8), np.ascontiguousarray(want).view(np.uint8))


def _codes(rng, shape, lo=-128, hi=127):
    return rng.integers(lo, hi + 1, size=shape).astype(np.int8)


CASES = [
    # (N, C, H, W, Cout, KH, KW, stride, pad, dilation, groups, mode)
    (2, 64, 14, 14, 64, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 0),      # ResNet body
    (2, 3, 32, 32, 64, 7, 7, (2, 2), (3, 3, 3, 3), (1, 1), 1, 0),       # ResNet stem, Cin 3
    (2, 64, 14, 14, 128, 1, 1, (2, 2), (0, 0, 0, 0), (1, 1), 1, 0),     # downsample 1x1/2
    (1, 32, 9, 11, 48, 3, 3, (1, 2), (1, 1, 2, 0), (2, 1), 2, 0),       # groups, dilation, asym pad
    (2, 32, 10, 10, 32, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 32, 0),     # depthwise
    (1, 20, 7, 7, 10, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 1),        # reflect, OHW 49
    (1, 20, 7, 9, 100, 5, 3, (1, 1), (2, 2, 1, 1), (1, 1), 1, 2),       # replicate
    (1, 17, 6, 6, 70, 3, 3, (2, 2), (1, 1, 1, 1), (1, 1), 1, 3),        # circular, ragged C
    (4, 64, 28, 28, 64, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 0),      # many pixel tiles
    (2, 256, 7, 7, 256, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 0),      # split K over 4
    (1, 512, 7, 7, 512, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1, 0),      # ResNet layer4: split K over 9
    (2, 256, 6, 6, 128, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 2, 0),      # split K with groups
    # tap-im2col form (2..4 channels per group, KW x Cg <= 32)
    (2, 4, 17, 19, 24, 3, 5, (1, 2), (1, 1, 2, 2), (1, 1), 1, 0),       # Cg 4, KW 5
    (1, 2, 12, 30, 16, 5, 9, (2, 3), (2, 2, 4, 4), (1, 2), 1, 1),       # Cg 2, reflect, dilated row
    (1, 6, 10, 10, 8, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 2, 2),        # Cg 3, two groups, replicate
    (1, 3, 9, 9, 5, 3, 7, (1, 1), (1, 1, 3, 3), (1, 1), 1, 3),          # circular, 21 taps x channels
    (1, 3, 5, 300, 8, 3, 3, (1, 2), (1, 1, 1, 1), (1, 1), 1, 0),        # 150 output columns: two blocks
    (3, 3, 1, 40, 12, 1, 5, (1, 1), (0, 0, 2, 2), (1, 1), 1, 0),        # a 1-D conv (height 1)
    (1, 6, 8, 16, 8, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 2, 0),         # Cg 3, two groups, zeros
    (1, 2, 12, 32, 16, 5, 9, (2, 3), (2, 2, 4, 4), (1, 2), 1, 0),       # Cg 2, dilated row, zeros
    (2, 3, 20, 260, 8, 7, 7, (2, 2), (3, 3, 3, 3), (1, 1), 1, 0),       # stem, 130 columns: two blocks
]


@pytest.mark.parametrize("case", CASES)
def test_conv_i8_exact(gpu, case):
    N, C, H, W, Cout, KH, KW, stride, pad, dil, groups, mode = case
    rng = np.random.default_rng(sum(case[:7]))
    x = _codes(rng, (N, C, H, W))
    w = _codes(rng, (Cout, C // groups, KH, KW), -127, 127)
    ws = rng.uniform(1e-3, 2e-2, Cout).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    kw = dict(stride=stride, pad=pad, dilation=dil, groups=groups, mode=mode, w_scale=ws, bias=b)
    for u8s8, za, relu in ((True, 131.0, True), (False, None, False), (False, -3.0, True)):
        got = run_conv(gpu, x, w, u8s8=u8s8, za=za, relu=relu, **kw)
        want = oracle_conv(x, w, u8s8=u8s8, za=za, relu=relu, **kw)
        _check(got, want, O.OUT_QU8S8)


@pytest.mark.parametrize("kind", [O.OUT_I32, O.OUT_F32, O.OUT_F16, O.OUT_Q8, O.OUT_QU8,
                                  O.OUT_FQ32, O.OUT_Q16, O.OUT_QU8S8])
def test_conv_i8_every_out_kind(gpu, kind):
    rng = np.random.default_rng(kind)
    x = _codes(rng, (2, 24, 9, 8))
    w = _codes(rng, (40, 24, 3, 3), -127, 127)
    qmin, qmax = GRID.get(kind, (-128, 127))
    kw = dict(u8s8=True, za=120.0, stride=(1, 1), pad=(1, 1, 1, 1), out_kind=kind, qmin=qmin,
              qmax=qmax, out_zp=(128.0 if qmin == 0 else -2.0), relu=True,
              bias=rng.standard_normal(40).astype(np.float32))
    _check(run_conv(gpu, x, w, **kw), oracle_conv(x, w, **kw), kind)


HALO_CASES = [
    # (N, C, H, W, Cout, KH, KW, pad): stride-1, zeros-padded convolutions with C = 64, Cout a
    # multiple of 64 and H * W % 16 == 0, which take the halo-staged kernel
    (8, 64, 56, 56, 64, 3, 3, (1, 1, 1, 1)),     # ResNet-18 layer1 at batch 8: tiles across images
    (3, 64, 28, 28, 128, 3, 3, (1, 1, 1, 1)),    # two output-channel blocks
    (6, 64, 12, 12, 64, 3, 3, (1, 1, 1, 1)),     # a tile spans 1.8 images
    (2, 64, 12, 20, 128, 3, 3, (0, 2, 1, 1)),    # asymmetric padding, ragged last tile
    (4, 64, 8, 10, 64, 2, 3, (1, 1, 0, 2)),      # non-square kernel, one-sided column padding
    (3, 64, 16, 36, 64, 3, 3, (1, 1, 1, 1)),     # rows that do not start on 16-byte chunks
]


@pytest.mark.parametrize("case", HALO_CASES)
@pytest.mark.parametrize("kind", [O.OUT_QU8S8, O.OUT_Q8, O.OUT_QU8])
def test_conv_halo_exact(gpu, case, kind):
    # the halo-staged kernel (input rows staged in LDS from the NCHW codes, no padded copy)
    # against the oracle's int64 convolution and epilogue, for each integer output kind,
    # with and without an activation zero point, ReLU and bias
    from lucid_amd import _C

    N, C, H, W, Cout, KH, KW, pad = case
    rng = np.random.default_rng(N * 1000 + C + H + Cout + kind)
    x = _codes(rng, (N, C, H, W))
    w = _codes(rng, (Cout, C, KH, KW), -127, 127)
    ws = rng.uniform(1e-3, 2e-2, Cout).astype(np.float32)
    qmin, qmax = GRID.get(kind, (-128, 127))
    zp = 128.0 if qmin == 0 else -3.0
    for u8s8, za, relu, bias in ((True, 131.0, True, True), (False, None, False, False), (False, -3.0, True, True)):
        kw = dict(stride=(1, 1), pad=pad, w_scale=ws, out_kind=kind, qmin=qmin, qmax=qmax, out_zp=zp,
                  bias=rng.standard_normal(Cout).astype(np.float32) if bias else None, a_scale=0.03,
                  out_scale=0.3)
        got = run_conv(gpu, x, w, u8s8=u8s8, za=za, relu=relu, **kw)
        assert _C.last_path() == "conv halo", _C.last_path()
        want = oracle_conv(x, w, u8s8=u8s8, za=za, relu=relu, **kw)
        _check(got, want, kind)


@pytest.mark.parametrize("case", [(2, 64, 16, 16, 64, 3, 3, (1, 1, 1, 1)), (2, 64, 14, 14, 128, 3, 3, (1, 1, 1, 1)),
                                  (2, 256, 7, 7, 256, 3, 3, (1, 1, 1, 1))])
@pytest.mark.parametrize("kind", [O.OUT_QU8S8, O.OUT_Q8, O.OUT_QU8])
def test_conv_epilogue_ties_exact(gpu, case, kind):
    # power-of-two scales, no bias and small codes put half the outputs on exact halves (ties
    # of the round-to-nearest-even) with an odd output zero point; the halo kernel, the 128 x 64
    # LDS-DMA tile and its split-K form against the oracle
    N, C, H, W, Cout, KH, KW, pad = case
    rng = np.random.default_rng(N * 1000 + C + H + Cout + kind + 17)
    x = _codes(rng, (N, C, H, W), -3, 3)
    w = _codes(rng, (Cout, C, KH, KW), -2, 2)
    qmin, qmax = GRID.get(kind, (-128, 127))
    zp = 127.0 if qmin == 0 else 3.0
    kw = dict(stride=(1, 1), pad=pad, w_scale=np.ones(Cout, np.float32), out_kind=kind, qmin=qmin, qmax=qmax,
              out_zp=zp, bias=None, a_scale=0.5, out_scale=1.0)
    print(f"conv ties {case} kind={kind}", flush=True)
    got = run_conv(gpu, x, w, **kw)
    want = oracle_conv(x, w, **kw)
    _check(got, want, kind)


def test_conv_halo_declines(gpu):
    # shapes outside the halo kernel's reach keep the packed-input kernels
    from lucid_amd import _C

    rng = np.random.default_rng(77)
    for (C, H, W, stride, kind) in ((64, 15, 14, (1, 1), O.OUT_QU8S8), (64, 16, 16, (2, 2), O.OUT_QU8S8),
                                    (48, 16, 16, (1, 1), O.OUT_QU8S8), (128, 16, 16, (1, 1), O.OUT_QU8S8),
                                    (64, 16, 16, (1, 1), O.OUT_F32)):
        x = _codes(rng, (4, C, H, W))
        w = _codes(rng, (64, C, 3, 3), -127, 127)
        kw = dict(stride=stride, pad=(1, 1, 1, 1), out_kind=kind)
        got = run_conv(gpu, x, w, **kw)
        assert _C.last_path() != "conv halo", (C, H, W, stride, kind)
        _check(got, oracle_conv(x, w, **kw), kind)


def test_conv_weight_pack_layout(gpu):
    rng = np.random.default_rng(4)
    w = _codes(rng, (10, 20, 3, 2))
    wp, sums = pack_conv_weights(gpu, w)
    Cp = 32
    want = np.zeros((10, 3, 2, Cp), np.int8)
    want[..., :20] = w.transpose(0, 2, 3, 1)
    rows = wp.numpy().reshape(10, 256)  # K = 3 * 2 * 32 = 192, rows padded to 256 bytes
    np.testing.assert_array_equal(rows[:, :192].reshape(10, 3, 2, Cp), want)
    assert not rows[:, 192:].any()
    np.testing.assert_array_equal(sums.numpy(), w.astype(np.int64).reshape(10, -1).sum(1))


def test_conv_weight_pack_taps_layout(gpu):
    """2..4 channels per group: rows [co][kh * 32 + kw * Cg + c], 32 bytes per kernel row."""
    rng = np.random.default_rng(5)
    w = _codes(rng, (10, 3, 7, 7))
    wp, sums = pack_conv_weights(gpu, w)
    rows = wp.numpy().reshape(10, 256)  # K = 7 * 32 = 224, rows padded to 256 bytes
    want = np.zeros((10, 7, 32), np.int8)
    want[:, :, :21] = w.transpose(0, 2, 3, 1).reshape(10, 7, 21)
    np.testing.assert_array_equal(rows[:, :224].reshape(10, 7, 32), want)
    assert not rows[:, 224:].any()
    np.testing.assert_array_equal(sums.numpy(), w.astype(np.int64).reshape(10, -1).sum(1))


def test_conv_rejects_bad_geometry(gpu):
    from lucid_amd import _C

    x = np.zeros((1, 4, 3, 3), np.int8)
    w = np.zeros((4, 4, 5, 5), np.int8)
    with pytest.raises(_C.LucidError, match="do not fit"):
        run_conv(gpu, x, w)
    with pytest.raises(_C.LucidError, match="smaller than the input"):
        run_conv(gpu, x, np.zeros((4, 4, 3, 3), np.int8), pad=(3, 3, 3, 3), mode=1)


@pytest.mark.parametrize("case", CASES[:6])
def test_conv_f32_exact(gpu, case):
    from lucid_amd import _C

    N, C, H, W, Cout, KH, KW, stride, pad, dil, groups, mode = case
    rng = np.random.default_rng(7 + sum(case[:7]))
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((Cout, C // groups, KH, KW)).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    OH, OW = O.conv_out_hw(H, W, KH, KW, stride, pad, dil)
    y = gpu.empty((N, Cout, OH, OW), np.float32, "gpu")
    xd, wd, bd = _dev(gpu, x), _dev(gpu, w), _dev(gpu, b)
    _C.call("lq_conv2d_f32", xd.data_ptr(), N, C, H, W, wd.data_ptr(), bd.data_ptr(), Cout, KH, KW,
            stride[0], stride[1], *pad, dil[0], dil[1], groups, mode, y.data_ptr(), None)
    want = O.conv2d_f32(x, w, b, stride=stride, pad=pad, dilation=dil, groups=groups, mode=mode)
    np.testing.assert_array_equal(y.numpy().view(np.uint32), want.view(np.uint32))


def test_batch_norm_f32_exact(gpu):
    from lucid_amd import _C

    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 5, 4, 3)).astype(np.float32)
    mean, var = rng.standard_normal(5).astype(np.float32), rng.uniform(0.5, 2, 5).astype(np.float32)
    gam, bet = rng.standard_normal(5).astype(np.float32), rng.standard_normal(5).astype(np.float32)
    y = gpu.empty(x.shape, np.float32, "gpu")
    d = [_dev(gpu, a) for a in (x, mean, var, gam, bet)]
    _C.call("lq_batch_norm_f32", d[0].data_ptr(), y.data_ptr(), 2, 5, 12, d[1].data_ptr(),
            d[2].data_ptr(), d[3].data_ptr(), d[4].data_ptr(), 1e-5, None)
    c = (slice(None), slice(None), None, None)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(1e-5))).astype(np.float32)
    want = ((((x - mean[c[1], None, None]) * inv[:, None, None]).astype(np.float32) * gam[:, None, None])
            .astype(np.float32) + bet[:, None, None]).astype(np.float32)
    np.testing.assert_array_equal(y.numpy(), want)
