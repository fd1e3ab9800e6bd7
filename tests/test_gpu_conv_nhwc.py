"""GPU parity of lq_conv2d_i8_nhwc -- the int8 convolution between activations held padded
NHWC (the layout its implicit GEMM reads), output written the same way with its border, and
the residual add_relu merge fused in -- against the NCHW path it stands for, bit for bit:
lq_conv2d_i8 on the NCHW codes, then lq_qmerge (LQ_MERGE_ADD, ReLU) with the skip codes.
Every ResNet-18 layer geometry at batch 2 (the small late layers split their K stages between
three wave groups of one workgroup, on 64 x 64 tiles), two and three groups on 128 x 64 tiles,
a cross-workgroup split-K plan, and a 1 x 1 stride-2 downsample reading a buffer bordered for a
3 x 3 consumer."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _d(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


def _nhwc(x, pad, fill):
    """NCHW int8 codes -> [N][H + 2 pad][W + 2 pad][C] with the border `fill`."""
    N, C, H, W = x.shape
    out = np.full((N, H + 2 * pad, W + 2 * pad, C), fill, np.int8)
    out[:, pad:pad + H, pad:pad + W, :] = x.transpose(0, 2, 3, 1)
    return out


CASES = [  # (C, Cout, H, k, stride, pad, x_pad, residual)
    (64, 64, 56, 3, 1, 1, 1, False), (64, 64, 56, 3, 1, 1, 1, True), (64, 128, 56, 3, 2, 1, 1, False),
    (64, 128, 56, 1, 2, 0, 1, False), (128, 128, 28, 3, 1, 1, 1, True), (256, 256, 14, 3, 1, 1, 1, True),
    (256, 512, 14, 3, 2, 1, 1, False), (512, 512, 7, 3, 1, 1, 1, True), (32, 48, 9, 3, 1, 1, 2, True),
    # K stages split between two wave groups (8 stages), three groups of 128 x 64 tiles (208
    # tiles), and a cross-workgroup split (25 stages)
    (1024, 64, 7, 1, 1, 0, 1, True), (128, 1024, 28, 3, 1, 1, 1, False), (128, 64, 9, 5, 1, 2, 2, True),
]


# Power-of-two scales and small codes: the convolution's outputs and the merge's sums land on
# exact halves (ties of the round-to-nearest-even), with odd zero points.
TIE_CASES = [(64, 64, 56, 3, 1, 1, 1, True, True), (128, 128, 28, 3, 1, 1, 1, True, True),
             (512, 512, 7, 3, 1, 1, 1, True, True)]


@pytest.mark.parametrize("C,Cout,H,k,stride,pad,x_pad,residual,ties", [c + (False,) for c in CASES] + TIE_CASES)
@pytest.mark.parametrize("y_pad", [1, 0])
def test_nhwc_conv_equals_the_nchw_path(gpu, C, Cout, H, k, stride, pad, x_pad, residual, ties, y_pad):
    from lucid_amd import _C

    lib = _C.lib()
    rng = np.random.default_rng(C + 7 * Cout + H + k + 3 * residual + 5 * ties)
    N = 2
    za, zo, zs, zm = (121.0, 9.0, 133.0, 5.0) if ties else (121.0, 9.0, 133.0, 4.0)
    if ties:
        x = rng.integers(-9, -4, (N, C, H, H)).astype(np.int8)  # codes 119..123 about za
        w = rng.integers(-2, 3, (Cout, C, k, k)).astype(np.int8)
    else:
        x = rng.integers(-128, 128, (N, C, H, H)).astype(np.int8)  # U8S8: code c stored as c - 128
        w = rng.integers(-127, 128, (Cout, C, k, k)).astype(np.int8)
    print(f"nhwc conv C={C} Cout={Cout} H={H} k={k} s={stride} residual={residual} ties={ties} y_pad={y_pad}",
          flush=True)
    dw = _d(gpu, w)
    wp = gpu.empty((lib.lq_conv2d_weight_pack_size(Cout, C, k, k),), np.int8, "gpu")
    sums = gpu.empty((Cout,), np.int32, "gpu")
    _C.call("lq_conv2d_pack_weights_i8", dw.data_ptr(), Cout, C, k, k, wp.data_ptr(), sums.data_ptr(), None)
    if ties:
        sa, sw = _d(gpu, np.float32(0.5)), _d(gpu, np.ones(Cout, np.float32))
        bias = _d(gpu, np.zeros(Cout, np.float32))
        so = _d(gpu, np.float32(1.0))
    else:
        sa, sw = _d(gpu, np.float32(0.02)), _d(gpu, rng.uniform(2e-4, 2e-3, Cout).astype(np.float32))
        bias = _d(gpu, (rng.standard_normal(Cout) * 0.3).astype(np.float32))
        so = _d(gpu, np.float32(0.03))
    dza, dzo = _d(gpu, np.float32(za)), _d(gpu, np.float32(zo))
    OH = (H + 2 * pad - k) // stride + 1
    # the NCHW path
    dx = _d(gpu, x)
    y_ref = gpu.empty((N, Cout, OH, OH), np.int8, "gpu")
    ws_n = max(lib.lq_conv2d_i8_workspace_size(N, C, H, H, Cout, k, k, stride, stride, pad, pad, pad, pad, 1, 1, 1), 16)
    ws = gpu.empty((ws_n,), np.uint8, "gpu")
    _C.call("lq_conv2d_i8", dx.data_ptr(), _C.U8S8, N, C, H, H, wp.data_ptr(), sums.data_ptr(), Cout, k, k, stride,
            stride, pad, pad, pad, pad, 1, 1, 1, 0, sa.data_ptr(), dza.data_ptr(), sw.data_ptr(), bias.data_ptr(),
            so.data_ptr(), dzo.data_ptr(), 0, 255, _C.OUT_QU8S8, _C.EPI_RELU if not residual else 0, y_ref.data_ptr(),
            ws.data_ptr(), ws_n, None)
    want = y_ref.numpy()
    skip = rng.integers(-128, 128, (N, Cout, OH, OH)).astype(np.int8)
    ss, sm = (_d(gpu, np.float32(0.5)), _d(gpu, np.float32(1.0))) if ties else \
        (_d(gpu, np.float32(0.025)), _d(gpu, np.float32(0.04)))
    dzs, dzm = _d(gpu, np.float32(zs)), _d(gpu, np.float32(zm))
    if residual:
        merged = gpu.empty((N * Cout * OH * OH,), np.int8, "gpu")
        _C.call("lq_qmerge", _C.MERGE_ADD, y_ref.data_ptr(), _C.U8S8, so.data_ptr(), dzo.data_ptr(),
                _d(gpu, skip).data_ptr(), _C.U8S8, ss.data_ptr(), dzs.data_ptr(), 0.0, 1, N * Cout * OH * OH,
                N * Cout * OH * OH, sm.data_ptr(), dzm.data_ptr(), 0, 255, _C.EPI_RELU, _C.U8S8, merged.data_ptr(),
                None)
        want = merged.numpy().reshape(N, Cout, OH, OH)
    # the NHWC path
    xp = _d(gpu, _nhwc(x, x_pad, np.int8(int(za) - 128)))
    zcode = np.int8(int(zm if residual else zo) - 128)
    yp = gpu.tensor(np.full((N, OH + 2 * y_pad, OH + 2 * y_pad, Cout), 0x5A, np.int8), device="gpu")
    dskip = _d(gpu, _nhwc(skip, y_pad, 0)) if residual else None
    nws = max(lib.lq_conv2d_i8_nhwc_workspace_size(N, C, H, H, Cout, k, k, stride, pad), 16)
    nw = gpu.empty((nws,), np.uint8, "gpu")
    _C.call("lq_conv2d_i8_nhwc", xp.data_ptr(), _C.U8S8, N, C, H, H, x_pad, C, wp.data_ptr(), sums.data_ptr(), Cout,
            k, k, stride, pad, sa.data_ptr(), dza.data_ptr(), sw.data_ptr(), bias.data_ptr(), so.data_ptr(),
            dzo.data_ptr(), 0, 255, _C.OUT_QU8S8, _C.EPI_RELU if not residual else 0, yp.data_ptr(), y_pad, Cout,
            dskip.data_ptr() if residual else None, _C.U8S8, ss.data_ptr(), dzs.data_ptr(), sm.data_ptr(),
            dzm.data_ptr(), 0, 255, _C.U8S8, _C.EPI_RELU, nw.data_ptr(), nws, None)
    path = _C.last_path()
    if (C, k) == (1024, 1) or Cout == 1024:
        assert path == "conv nhwc dma 128x64 wave-group split-k", path
    if (C, k) == (512, 3):
        assert path == "conv nhwc dma 64x64 wave-group split-k", path
    if (C, k) == (128, 5):
        assert path == "conv nhwc dma 128x64 split-k", path
    got = yp.numpy()
    np.testing.assert_array_equal(got[:, y_pad:y_pad + OH, y_pad:y_pad + OH, :], want.transpose(0, 2, 3, 1))
    if y_pad:
        border = np.ones(got.shape[:3], bool)
        border[:, 1:-1, 1:-1] = False
        assert np.all(got[border] == zcode)


@pytest.mark.parametrize("N,C,H,k,stride,pad,y_pad,code", [(2, 64, 112, 3, 2, 1, 1, "U8S8"), (3, 32, 17, 3, 2, 1, 1, "U8"),
                                                           (1, 64, 9, 2, 2, 0, 0, "I8"), (2, 128, 20, 3, 1, 1, 1, "I8")])
def test_maxpool_to_nhwc_equals_lq_pool2d(gpu, N, C, H, k, stride, pad, y_pad, code):
    from lucid_amd import _C

    rng = np.random.default_rng(N * C + H)
    t = getattr(_C, code)
    x = (rng.integers(0, 256, (N, C, H, H)).astype(np.uint8) if code == "U8"
         else rng.integers(-128, 128, (N, C, H, H)).astype(np.int8))
    OH = (H + 2 * pad - k) // stride + 1
    dx = _d(gpu, x)
    ref = gpu.empty((N, C, OH, OH), x.dtype, "gpu")
    _C.call("lq_pool2d", _C.POOL_MAX, dx.data_ptr(), t, None, None, N, C, H, H, OH, OH, k, k, stride, stride, pad, pad,
            0, ref.data_ptr(), None)
    zp = 77.0
    yp = gpu.tensor(np.full((N, OH + 2 * y_pad, OH + 2 * y_pad, C), 0x33, np.int8), device="gpu")
    _C.call("lq_maxpool2d_i8_to_nhwc", dx.data_ptr(), t, _d(gpu, np.float32(zp)).data_ptr(), N, C, H, H, OH, OH, k, k,
            stride, stride, pad, pad, yp.data_ptr(), y_pad, C, None)
    got = yp.numpy()
    want = ref.numpy().view(np.int8).transpose(0, 2, 3, 1)
    np.testing.assert_array_equal(got[:, y_pad:y_pad + OH, y_pad:y_pad + OH, :], want)
    if y_pad:
        border = np.ones(got.shape[:3], bool)
        border[:, 1:-1, 1:-1] = False
        zc = np.int8(int(zp) - 128) if code == "U8S8" else np.uint8(int(zp)).view(np.int8)
        assert np.all(got[border] == zc)


@pytest.mark.parametrize("N,C,H,x_pad,code", [(2, 512, 7, 1, "U8S8"), (3, 48, 5, 0, "U8"), (2, 64, 56, 1, "I8")])
def test_global_avgpool_nhwc_equals_lq_pool2d(gpu, N, C, H, x_pad, code):
    from lucid_amd import _C

    rng = np.random.default_rng(C + H)
    t = getattr(_C, code)
    x = (rng.integers(0, 256, (N, C, H, H)).astype(np.uint8) if code == "U8"
         else rng.integers(-128, 128, (N, C, H, H)).astype(np.int8))
    s, z = _d(gpu, np.float32(0.037)), _d(gpu, np.float32(11.0))
    ref = gpu.empty((N, C, 1, 1), np.float32, "gpu")
    _C.call("lq_pool2d", _C.POOL_AVG, _d(gpu, x).data_ptr(), t, s.data_ptr(), z.data_ptr(), N, C, H, H, 1, 1, 0, 0,
            0, 0, 0, 0, _C.POOL_ADAPTIVE, ref.data_ptr(), None)
    xp = _d(gpu, _nhwc(x.view(np.int8), x_pad, 0))
    y = gpu.empty((N, C), np.float32, "gpu")
    _C.call("lq_avgpool2d_global_nhwc", xp.data_ptr(), t, s.data_ptr(), z.data_ptr(), N, C, H, H, x_pad, C,
            y.data_ptr(), None)
    np.testing.assert_array_equal(y.numpy().view(np.uint32), ref.numpy().reshape(N, C).view(np.uint32))


@pytest.mark.parametrize("C,Cout,H,k,stride,pad", [(3, 64, 224, 7, 2, 3), (64, 128, 28, 3, 1, 1), (16, 32, 12, 1, 1, 0)])
def test_conv_out_nhwc_flag_is_the_nchw_output_transposed(gpu, C, Cout, H, k, stride, pad):
    """lq_conv2d_i8 with LQ_CONV_OUT_NHWC (the ResNet stem's tap-im2col form among them) writes
    the NCHW call's codes as [N][OH][OW][Cout]."""
    from lucid_amd import _C

    lib = _C.lib()
    rng = np.random.default_rng(C * Cout + H)
    N = 2
    x = _d(gpu, rng.integers(-128, 128, (N, C, H, H)).astype(np.int8))
    w = _d(gpu, rng.integers(-127, 128, (Cout, C, k, k)).astype(np.int8))
    wp = gpu.empty((lib.lq_conv2d_weight_pack_size(Cout, C, k, k),), np.int8, "gpu")
    sums = gpu.empty((Cout,), np.int32, "gpu")
    _C.call("lq_conv2d_pack_weights_i8", w.data_ptr(), Cout, C, k, k, wp.data_ptr(), sums.data_ptr(), None)
    OH = (H + 2 * pad - k) // stride + 1
    ws_n = max(lib.lq_conv2d_i8_workspace_size(N, C, H, H, Cout, k, k, stride, stride, pad, pad, pad, pad, 1, 1, 1), 16)
    ws = gpu.empty((ws_n,), np.uint8, "gpu")
    sa, za = _d(gpu, np.float32(0.02)), _d(gpu, np.float32(100.0))
    sw = _d(gpu, rng.uniform(1e-4, 1e-3, Cout).astype(np.float32))
    so, zo = _d(gpu, np.float32(0.05)), _d(gpu, np.float32(3.0))
    outs = []
    for flags in (_C.EPI_RELU, _C.EPI_RELU | _C.CONV_OUT_NHWC):
        y = gpu.empty((N * Cout * OH * OH,), np.int8, "gpu")
        _C.call("lq_conv2d_i8", x.data_ptr(), _C.U8S8, N, C, H, H, wp.data_ptr(), sums.data_ptr(), Cout, k, k, stride,
                stride, pad, pad, pad, pad, 1, 1, 1, 0, sa.data_ptr(), za.data_ptr(), sw.data_ptr(), None,
                so.data_ptr(), zo.data_ptr(), 0, 255, _C.OUT_QU8S8, flags, y.data_ptr(), ws.data_ptr(), ws_n, None)
        outs.append(y.numpy())
    np.testing.assert_array_equal(outs[1].reshape(N, OH, OH, Cout), outs[0].reshape(N, Cout, OH, OH).transpose(0, 2, 3, 1))


@pytest.mark.parametrize("N,C,H,x_pad,y_pad,code", [(2, 64, 112, 0, 1, "U8S8"), (3, 32, 15, 1, 0, "U8"), (1, 16, 8, 2, 1, "I8")])
def test_maxpool_nhwc_equals_lq_pool2d(gpu, N, C, H, x_pad, y_pad, code):
    from lucid_amd import _C

    rng = np.random.default_rng(N + C + H)
    t = getattr(_C, code)
    x = (rng.integers(0, 256, (N, C, H, H)).astype(np.uint8) if code == "U8"
         else rng.integers(-128, 128, (N, C, H, H)).astype(np.int8))
    OH = (H + 2 - 3) // 2 + 1
    ref = gpu.empty((N, C, OH, OH), x.dtype, "gpu")
    _C.call("lq_pool2d", _C.POOL_MAX, _d(gpu, x).data_ptr(), t, None, None, N, C, H, H, OH, OH, 3, 3, 2, 2, 1, 1, 0,
            ref.data_ptr(), None)
    zp = 5.0
    xp = _d(gpu, _nhwc(x.view(np.int8), x_pad, 99))
    yp = gpu.tensor(np.full((N, OH + 2 * y_pad, OH + 2 * y_pad, C), 0x33, np.int8), device="gpu")
    _C.call("lq_maxpool2d_i8_nhwc", xp.data_ptr(), t, _d(gpu, np.float32(zp)).data_ptr(), N, C, H, H, x_pad, C, OH,
            OH, 3, 3, 2, 2, 1, 1, yp.data_ptr(), y_pad, C, None)
    got = yp.numpy()
    np.testing.assert_array_equal(got[:, y_pad:y_pad + OH, y_pad:y_pad + OH, :],
                                  ref.numpy().view(np.int8).transpose(0, 2, 3, 1))
    if y_pad:
        border = np.ones(got.shape[:3], bool)
        border[:, 1:-1, 1:-1] = False
        zc = np.int8(int(zp) - 128) if code == "U8S8" else np.int8(int(zp))
        assert np.all(got[border] == zc)
