"""GPU parity of the decoder glue kernels (lucid_amd/csrc/lq_glue.hip) through the C ABI:
embedding sums, residual adds, the KV-cache append and argmax bit-exact; layer norm and the
tanh GELU within fp32 rtol 1e-5 of the oracle's float64; attention (fp16 q / k / v, fp32
scores and sums) within rtol 1e-4 of float64 over the same fp16 values, at prefill and
decode positions, with the position passed by value and through a device counter."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from _tolerance import assert_close_f32, assert_close_to_scale

pytestmark = pytest.mark.gpu


def _d(L, a):
    return L.tensor(np.ascontiguousarray(a), device="gpu")


def test_embedding_sum_and_add_exact(gpu):
    from lucid_amd import _C

    rng = np.random.default_rng(1)
    V, P, D, B, n, pos0 = 1000, 64, 48, 3, 5, 7
    tok = rng.standard_normal((V, D)).astype(np.float32)
    pos = rng.standard_normal((P, D)).astype(np.float32)
    ids = rng.integers(0, V, (B, n)).astype(np.int32)
    out = gpu.empty((B * n, D), np.float32, "gpu")
    dt, dp, di = _d(gpu, tok), _d(gpu, pos), _d(gpu, ids)
    _C.call("lq_embedding_sum_f32", dt.data_ptr(), V, dp.data_ptr(), P, D, di.data_ptr(), B * n, n, pos0, None,
            out.data_ptr(), None)
    want = O.embedding_sum(tok, pos, ids, pos0).reshape(B * n, D)
    np.testing.assert_array_equal(out.numpy(), want)
    dpos = _d(gpu, np.array([pos0 + 3], np.int32))  # device position
    _C.call("lq_embedding_sum_f32", dt.data_ptr(), V, dp.data_ptr(), P, D, di.data_ptr(), B * n, n, 0,
            dpos.data_ptr(), out.data_ptr(), None)
    np.testing.assert_array_equal(out.numpy(), O.embedding_sum(tok, pos, ids, pos0 + 3).reshape(B * n, D))
    a, b = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    y = gpu.empty((1000,), np.float32, "gpu")
    da, db = _d(gpu, a), _d(gpu, b)
    _C.call("lq_add_f32", da.data_ptr(), db.data_ptr(), y.data_ptr(), 1000, None)
    np.testing.assert_array_equal(y.numpy(), a + b)
    _C.call("lq_increment_i32", dpos.data_ptr(), 5, None)
    assert dpos.numpy()[0] == pos0 + 8


@pytest.mark.parametrize("rows,D", [(8, 512), (4096, 512), (9, 100), (6, 2048)])
def test_add_layer_norm_matches_add_then_norm(gpu, rows, D):
    """lq_add_layer_norm_f32 (x += res, then the norm of x) gives the bits of lq_add_f32
    followed by lq_layer_norm_f32, for the updated residual stream and for the norm, with and
    without gamma / beta and with strided rows."""
    from lucid_amd import _C

    rng = np.random.default_rng(rows * 7 + D)
    x = (rng.standard_normal((rows, D)) * 2 + 0.5).astype(np.float32)
    res = rng.standard_normal((rows, 2 * D)).astype(np.float32)  # rows 2 D apart, the first D used
    g, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    dg, dbb = _d(gpu, g), _d(gpu, b)
    dres = _d(gpu, res)
    rc = _d(gpu, np.ascontiguousarray(res[:, :D]))
    for gamma, beta in ((None, None), (dg.data_ptr(), dbb.data_ptr())):
        xa, xb = _d(gpu, x), _d(gpu, x)
        ya = gpu.empty((rows, D), np.float32, "gpu")
        yb = gpu.empty((rows, 3 * D), np.float32, "gpu")
        _C.call("lq_add_f32", xa.data_ptr(), rc.data_ptr(), xa.data_ptr(), rows * D, None)
        _C.call("lq_layer_norm_f32", xa.data_ptr(), D, ya.data_ptr(), D, rows, D, gamma, beta, np.float32(1e-5),
                None)
        _C.call("lq_add_layer_norm_f32", xb.data_ptr(), D, dres.data_ptr(), 2 * D, yb.data_ptr(), 3 * D, rows, D,
                gamma, beta, np.float32(1e-5), None)
        np.testing.assert_array_equal(xb.numpy().view(np.uint32), xa.numpy().view(np.uint32))
        np.testing.assert_array_equal(yb.numpy()[:, :D].view(np.uint32), ya.numpy().view(np.uint32))
        want = x + res[:, :D]
        np.testing.assert_array_equal(xb.numpy(), want)
        assert_close_f32(yb.numpy()[:, :D], O.layer_norm(want, None if gamma is None else g,
                                                          None if beta is None else b, 1e-5))


@pytest.mark.parametrize("rows,D", [(1, 512), (4096, 512), (9, 100), (3, 2048)])
def test_layer_norm(gpu, rows, D):
    from lucid_amd import _C

    rng = np.random.default_rng(rows + D)
    x = (rng.standard_normal((rows, D)) * 2 + 0.5).astype(np.float32)
    g, b = rng.standard_normal(D).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    dx, dg, dbb = _d(gpu, x), _d(gpu, g), _d(gpu, b)
    y = gpu.empty((rows, D), np.float32, "gpu")
    _C.call("lq_layer_norm_f32", dx.data_ptr(), D, y.data_ptr(), D, rows, D, None, None, np.float32(1e-5), None)
    assert_close_f32(y.numpy(), O.layer_norm(x, eps=1e-5))
    _C.call("lq_layer_norm_f32", dx.data_ptr(), D, y.data_ptr(), D, rows, D, dg.data_ptr(), dbb.data_ptr(),
            np.float32(1e-5), None)
    assert_close_f32(y.numpy(), O.layer_norm(x, g, b, 1e-5))
    if rows >= 3:  # strided rows: every third row, packed output
        k = rows // 3
        y2 = gpu.empty((k, D), np.float32, "gpu")
        _C.call("lq_layer_norm_f32", dx.data_ptr() + 2 * D * 4, 3 * D, y2.data_ptr(), D, k, D, None, None,
                np.float32(1e-5), None)
        assert_close_f32(y2.numpy(), O.layer_norm(x[2::3][:k], eps=1e-5))


def test_gelu_tanh(gpu):
    from lucid_amd import _C

    x = np.concatenate([np.linspace(-10, 10, 4001), np.random.default_rng(2).standard_normal(10000) * 3]).astype(np.float32)
    y = gpu.empty(x.shape, np.float32, "gpu")
    dx = _d(gpu, x)
    _C.call("lq_gelu_tanh_f32", dx.data_ptr(), y.data_ptr(), x.size, None)
    assert_close_f32(y.numpy(), O.gelu_tanh(x))


def _attention_case(gpu, B, H, n, pos0, T_max, device_pos):
    from lucid_amd import _C

    hd = 64
    rng = np.random.default_rng(B * 100 + n + pos0)
    qkv = rng.standard_normal((B, n, 3, H, hd)).astype(np.float32)
    kc = np.zeros((B, H, T_max, hd), np.float16)
    vc = np.zeros((B, H, T_max, hd), np.float16)
    kc[:, :, :pos0] = rng.standard_normal((B, H, pos0, hd))  # earlier positions already cached
    vc[:, :, :pos0] = rng.standard_normal((B, H, pos0, hd))
    dqkv, dk, dv = _d(gpu, qkv), _d(gpu, kc), _d(gpu, vc)
    dq = gpu.empty((B, H, n, hd), np.float16, "gpu")
    dpos = _d(gpu, np.array([pos0], np.int32)) if device_pos else None
    p0 = 0 if device_pos else pos0
    pptr = dpos.data_ptr() if device_pos else None
    _C.call("lq_kv_append_f16", dqkv.data_ptr(), B, n, H, hd, p0, pptr, T_max, dq.data_ptr(), dk.data_ptr(),
            dv.data_ptr(), None)
    q16 = qkv[:, :, 0].transpose(0, 2, 1, 3).astype(np.float16)
    np.testing.assert_array_equal(dq.numpy().view(np.uint16), q16.view(np.uint16))
    kc[:, :, pos0:pos0 + n] = qkv[:, :, 1].transpose(0, 2, 1, 3).astype(np.float16)
    vc[:, :, pos0:pos0 + n] = qkv[:, :, 2].transpose(0, 2, 1, 3).astype(np.float16)
    np.testing.assert_array_equal(dk.numpy().view(np.uint16), kc.view(np.uint16))
    np.testing.assert_array_equal(dv.numpy().view(np.uint16), vc.view(np.uint16))
    out = gpu.empty((B, n, H, hd), np.float32, "gpu")
    scale = np.float32(1.0 / 8.0)
    _C.call("lq_attention_f16", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H, n, hd, p0, pptr, T_max,
            scale, out.data_ptr(), None)
    assert_close_to_scale(out.numpy(), O.attention(q16, kc, vc, pos0, scale), 1e-4)


@pytest.mark.parametrize("B,H,n,pos0,T_max", [(2, 3, 40, 0, 64), (8, 8, 512, 0, 640), (8, 8, 1, 511, 640),
                                              (8, 8, 1, 639, 640), (1, 2, 9, 100, 2048), (2, 1, 1, 0, 16),
                                              (2, 3, 70, 5, 80), (1, 1, 130, 3000, 3200), (3, 2, 64, 0, 64),
                                              (1, 1, 1, 2047, 2048)])
def test_kv_append_and_attention(gpu, B, H, n, pos0, T_max):
    print(f"attention B={B} H={H} n={n} pos0={pos0}", flush=True)
    _attention_case(gpu, B, H, n, pos0, T_max, device_pos=False)
    _attention_case(gpu, B, H, n, pos0, T_max, device_pos=True)


@pytest.mark.parametrize("hd,off", [(8, 0), (24, 0), (12, 0), (64, 1)])
def test_kv_append_head_dims(gpu, hd, off):
    """lq_kv_append_f16 at head dims other than attention's 64: eight dims per lane when hd % 8
    == 0 and the buffers are 16-byte aligned, element by element otherwise (hd 12, or a qkv
    buffer one float past alignment) -- the same fp16 bits either way."""
    from lucid_amd import _C

    B, n, H, T_max, pos0 = 2, 5, 3, 9, 4
    rng = np.random.default_rng(hd)
    qkv = (rng.standard_normal((B, n, 3, H, hd)) * 100).astype(np.float32)
    qkv.flat[::7] = np.float32(65520.0)  # rounds to infinity in fp16
    buf = _d(gpu, np.concatenate([np.zeros(off, np.float32), qkv.ravel()]))
    kc = np.zeros((B, H, T_max, hd), np.float16)
    vc = np.zeros((B, H, T_max, hd), np.float16)
    dk, dv = _d(gpu, kc), _d(gpu, vc)
    dq = gpu.empty((B, H, n, hd), np.float16, "gpu")
    _C.call("lq_kv_append_f16", buf.data_ptr() + 4 * off, B, n, H, hd, pos0, None, T_max, dq.data_ptr(),
            dk.data_ptr(), dv.data_ptr(), None)
    q16 = qkv[:, :, 0].transpose(0, 2, 1, 3).astype(np.float16)
    kc[:, :, pos0:pos0 + n] = qkv[:, :, 1].transpose(0, 2, 1, 3).astype(np.float16)
    vc[:, :, pos0:pos0 + n] = qkv[:, :, 2].transpose(0, 2, 1, 3).astype(np.float16)
    np.testing.assert_array_equal(dq.numpy().view(np.uint16), q16.view(np.uint16))
    np.testing.assert_array_equal(dk.numpy().view(np.uint16), kc.view(np.uint16))
    np.testing.assert_array_equal(dv.numpy().view(np.uint16), vc.view(np.uint16))


@pytest.mark.parametrize("B,n,H,pos0,T_max", [(8, 512, 8, 0, 640), (2, 37, 3, 5, 64), (1, 1, 1, 10, 16)])
def test_kv_append_from_fp16_equals_float(gpu, B, n, H, pos0, T_max):
    """lq_kv_append_h16 on qkv rounded to fp16 writes q and the caches with the bits
    lq_kv_append_f16 writes from the float32 qkv (the prefill's projection rounds in its
    epilogue); a misaligned or hd % 8 != 0 call is refused."""
    from lucid_amd import _C

    hd = 64
    rng = np.random.default_rng(B * 1000 + n)
    qkv = (rng.standard_normal((B, n, 3, H, hd)) * 4).astype(np.float32)
    qkv.flat[::11] = np.float32(70000.0)  # overflows fp16 to infinity in both routes
    outs = []
    for src in (qkv, qkv.astype(np.float16)):
        kc = np.full((B, H, T_max, hd), 0.5, np.float16)
        dk, dv = _d(gpu, kc), _d(gpu, kc)
        dq = gpu.empty((B, H, n, hd), np.float16, "gpu")
        fn = "lq_kv_append_f16" if src.dtype == np.float32 else "lq_kv_append_h16"
        _C.call(fn, _d(gpu, src).data_ptr(), B, n, H, hd, pos0, None, T_max, dq.data_ptr(), dk.data_ptr(),
                dv.data_ptr(), None)
        outs.append([t.numpy().view(np.uint16) for t in (dq, dk, dv)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    with pytest.raises(_C.LucidError, match="multiple of 8"):
        _C.call("lq_kv_append_h16", 16, 1, 1, 1, 12, 0, None, 4, 16, 16, 16, None)


@pytest.mark.parametrize("B,H,n,pos0,T_max,qoff", [(8, 8, 512, 0, 640, 0), (1, 2, 130, 3, 200, 0),
                                                   (2, 3, 70, 5, 80, 0), (2, 3, 40, 0, 64, 0),
                                                   (8, 8, 512, 0, 640, 1), (8, 8, 1, 511, 640, 0)])
def test_attention_dynamic_quantize_equals_calls(gpu, B, H, n, pos0, T_max, qoff):
    """lq_attention_dynamic_quantize_f16: the attention output, the codes and the qparams bit for
    bit those of lq_attention_f16 followed by lq_dynamic_quantize_f32 (two launches for the
    flash kernel above 16384 values with aligned codes; otherwise the calls: 15360 values, codes
    one byte past alignment, a single query)."""
    from lucid_amd import _C

    print(f"attention dynamic quantize B={B} H={H} n={n} pos0={pos0} qoff={qoff}", flush=True)
    hd = 64
    rng = np.random.default_rng(B * 10 + n)
    q = rng.standard_normal((B, H, n, hd)).astype(np.float16)
    kc = rng.standard_normal((B, H, T_max, hd)).astype(np.float16)
    vc = (rng.standard_normal((B, H, T_max, hd)) * 3).astype(np.float16)
    dq, dk, dv = _d(gpu, q), _d(gpu, kc), _d(gpu, vc)
    total = B * n * H * hd
    scale, eps = np.float32(0.125), np.float32(1e-8)
    o1, o2 = gpu.empty((B, n, H, hd), np.float32, "gpu"), gpu.empty((B, n, H, hd), np.float32, "gpu")
    c1, c2 = gpu.empty((total,), np.int8, "gpu"), gpu.empty((total + 16,), np.int8, "gpu")
    p1, p2 = gpu.empty((4,), np.float32, "gpu"), gpu.empty((4,), np.float32, "gpu")
    ws1_n = max(_C.lib().lq_dynamic_quantize_workspace_size(total), 16)
    ws1 = gpu.empty((ws1_n,), np.uint8, "gpu")
    _C.call("lq_attention_f16", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H, n, hd, pos0, None, T_max, scale,
            o1.data_ptr(), None)
    _C.call("lq_dynamic_quantize_f32", o1.data_ptr(), total, _C.U8S8, 0, 255, eps, p1.data_ptr(), c1.data_ptr(),
            ws1.data_ptr(), ws1_n, None)
    ws2_n = _C.lib().lq_attention_dynamic_quantize_workspace_size(B, H, n, hd)
    ws2 = gpu.empty((max(ws2_n, 16),), np.uint8, "gpu")
    _C.call("lq_attention_dynamic_quantize_f16", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H, n, hd, pos0,
            None, T_max, scale, o2.data_ptr(), _C.U8S8, 0, 255, eps, p2.data_ptr(), c2.data_ptr() + qoff,
            ws2.data_ptr(), ws2_n, None)
    two = n > 1 and total > 16384 and not qoff
    want = ("attention dynamic quantize two-launch" if two
            else "dynamic quantize fused" if total <= 16384 else "dynamic quantize")
    assert _C.last_path() == want
    np.testing.assert_array_equal(o1.numpy().view(np.uint32), o2.numpy().view(np.uint32))
    np.testing.assert_array_equal(c1.numpy(), c2.numpy()[qoff:qoff + total])
    np.testing.assert_array_equal(p1.numpy().view(np.uint32), p2.numpy().view(np.uint32))
    ov = o2.numpy()
    np.testing.assert_array_equal(p2.numpy()[:2], np.array([ov.min(), ov.max()], np.float32))


def test_attention_rejects_unsupported(gpu):
    from lucid_amd import _C

    with pytest.raises(_C.LucidError, match="head dim"):
        _C.call("lq_attention_f16", 1, 1, 1, 1, 1, 1, 32, 0, None, 4, np.float32(1.0), 1, None)
    with pytest.raises(_C.LucidError, match="2048"):
        _C.call("lq_attention_f16", 1, 1, 1, 1, 1, 1, 64, 2048, None, 4096, np.float32(1.0), 1, None)
    with pytest.raises(_C.LucidError, match="2048"):
        _C.call("lq_kv_append_attention_f16", 1, 1, 1, 64, 2048, None, 4096, 1, 1, np.float32(1.0), 1, None)


def test_argmax(gpu):
    from lucid_amd import _C

    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 32000)).astype(np.float32)
    x[1, [5, 900, 31999]] = 50.0          # ties: first index
    x[2, 17] = np.nan                     # NaN wins
    x[3, [40, 41]] = np.nan               # first NaN
    x[4] = -np.inf
    x[5, 31999] = np.inf
    idx = gpu.empty((9,), np.int32, "gpu")
    dx = _d(gpu, x)
    _C.call("lq_argmax_f32", dx.data_ptr(), 9, 32000, idx.data_ptr(), None)
    np.testing.assert_array_equal(idx.numpy(), np.argmax(x, axis=1))
    # the same with the position advance fused in; ragged widths take the scalar loads
    pos = _d(gpu, np.array([7], np.int32))
    _C.call("lq_argmax_next_f32", dx.data_ptr(), 9, 32000, idx.data_ptr(), pos.data_ptr(), 3, None)
    np.testing.assert_array_equal(idx.numpy(), np.argmax(x, axis=1))
    assert pos.numpy()[0] == 10
    for cols in (1, 5, 1023, 4097, 33333):
        y = rng.standard_normal((3, cols)).astype(np.float32)
        y[0, cols // 2] = np.nan
        y[1, -1] = y[1].max() + 1.0
        y[2, :] = 0.5  # all tied: index 0
        dy = _d(gpu, y)
        _C.call("lq_argmax_f32", dy.data_ptr(), 3, cols, idx.data_ptr(), None)
        np.testing.assert_array_equal(idx.numpy()[:3], np.argmax(y, axis=1), err_msg=f"cols={cols}")


def test_kv_append_attention_fused_equals_two_calls(gpu):
    """The decode step's fused append + attention: the caches and the output bit for bit those
    of lq_kv_append_f16 followed by lq_attention_f16 (n = 1), with the position by value and
    from the device counter."""
    from lucid_amd import _C

    B, H, hd, T_max = 8, 8, 64, 640
    rng = np.random.default_rng(31)
    for pos0, device_pos in ((0, False), (511, True), (639, False)):
        qkv = rng.standard_normal((B, 1, 3, H, hd)).astype(np.float32)
        kc = rng.standard_normal((B, H, T_max, hd)).astype(np.float16)
        vc = rng.standard_normal((B, H, T_max, hd)).astype(np.float16)
        dqkv = _d(gpu, qkv)
        k1, v1, k2, v2 = _d(gpu, kc), _d(gpu, vc), _d(gpu, kc), _d(gpu, vc)
        dpos = _d(gpu, np.array([pos0], np.int32))
        p0, pp = (0, dpos.data_ptr()) if device_pos else (pos0, None)
        dq = gpu.empty((B, H, 1, hd), np.float16, "gpu")
        o1, o2 = gpu.empty((B, 1, H, hd), np.float32, "gpu"), gpu.empty((B, 1, H, hd), np.float32, "gpu")
        scale = np.float32(0.125)
        _C.call("lq_kv_append_f16", dqkv.data_ptr(), B, 1, H, hd, p0, pp, T_max, dq.data_ptr(), k1.data_ptr(),
                v1.data_ptr(), None)
        _C.call("lq_attention_f16", dq.data_ptr(), k1.data_ptr(), v1.data_ptr(), B, H, 1, hd, p0, pp, T_max, scale,
                o1.data_ptr(), None)
        _C.call("lq_kv_append_attention_f16", dqkv.data_ptr(), B, H, hd, p0, pp, T_max, k2.data_ptr(), v2.data_ptr(),
                scale, o2.data_ptr(), None)
        np.testing.assert_array_equal(k1.numpy().view(np.uint16), k2.numpy().view(np.uint16))
        np.testing.assert_array_equal(v1.numpy().view(np.uint16), v2.numpy().view(np.uint16))
        np.testing.assert_array_equal(o1.numpy().view(np.uint32), o2.numpy().view(np.uint32))


@pytest.mark.parametrize("rows,D,with_res", [(8, 512, False), (8, 512, True), (3, 700, True), (24, 512, True),
                                             (1, 12288, False)])
def test_layer_norm_quantize_equals_two_calls(gpu, rows, D, with_res):
    """lq_layer_norm_quantize_f32: x (after x += res), the codes and the qparams bit for bit
    those of lq_(add_)layer_norm_f32 followed by lq_dynamic_quantize_f32 on the unsigned grid
    stored as c - 128 (the dynamic Linear's input)."""
    from lucid_amd import _C

    rng = np.random.default_rng(rows * 7 + D)
    x = (rng.standard_normal((rows, D)) * 3 + 1).astype(np.float32)
    r = rng.standard_normal((rows, D)).astype(np.float32)
    x1, x2, dr = _d(gpu, x), _d(gpu, x), _d(gpu, r)
    y = gpu.empty((rows, D), np.float32, "gpu")
    q1, q2 = gpu.empty((rows * D,), np.int8, "gpu"), gpu.empty((rows * D,), np.int8, "gpu")
    qp1, qp2 = gpu.empty((4,), np.float32, "gpu"), gpu.empty((4,), np.float32, "gpu")
    eps_ln, eps = np.float32(1e-5), np.float32(1e-8)
    ws_n = _C.lib().lq_dynamic_quantize_workspace_size(rows * D)
    ws = gpu.empty((max(ws_n, 16),), np.uint8, "gpu")
    if with_res:
        _C.call("lq_add_layer_norm_f32", x1.data_ptr(), D, dr.data_ptr(), D, y.data_ptr(), D, rows, D, None, None,
                eps_ln, None)
    else:
        _C.call("lq_layer_norm_f32", x1.data_ptr(), D, y.data_ptr(), D, rows, D, None, None, eps_ln, None)
    _C.call("lq_dynamic_quantize_f32", y.data_ptr(), rows * D, _C.U8S8, 0, 255, eps, qp1.data_ptr(), q1.data_ptr(),
            ws.data_ptr(), ws_n, None)
    _C.call("lq_layer_norm_quantize_f32", x2.data_ptr(), D, dr.data_ptr() if with_res else None, D, rows, D, None,
            None, eps_ln, _C.U8S8, 0, 255, eps, qp2.data_ptr(), q2.data_ptr(), None)
    np.testing.assert_array_equal(x1.numpy().view(np.uint32), x2.numpy().view(np.uint32))
    np.testing.assert_array_equal(q1.numpy(), q2.numpy())
    np.testing.assert_array_equal(qp1.numpy().view(np.uint32), qp2.numpy().view(np.uint32))
    # and the norm itself against float64 (the codes' source)
    xr = x + r if with_res else x
    sc, zp = qp2.numpy()[2], qp2.numpy()[3]
    codes = q2.numpy().astype(np.int64) + 128
    deq = (codes - zp) * sc
    assert np.max(np.abs(deq - O.layer_norm(xr).ravel())) <= sc * 0.5 + 1e-4


@pytest.mark.parametrize("rows,D,with_res,affine,qoff", [
    (4096, 512, True, False, 0), (4096, 512, False, True, 0), (5000, 700, True, True, 0), (33, 2560, True, False, 0),
    (4099, 256, False, False, 0), (8, 512, True, False, 0), (6, 3001, True, True, 1)])
def test_layer_norm_dynamic_quantize_equals_calls(gpu, rows, D, with_res, affine, qoff):
    """lq_layer_norm_dynamic_quantize_f32: x (after x += res), the normalized rows y, the codes and
    the qparams bit for bit those of lq_(add_)layer_norm_f32 followed by lq_dynamic_quantize_f32
    (two launches above 16384 values with aligned buffers -- 5000 rows fold more rows than
    workgroups, D 2560 takes the wide norm -- else the separate calls: 4096 values, or codes one
    byte past alignment)."""
    from lucid_amd import _C

    print(f"ln dynamic quantize rows={rows} D={D} res={with_res}", flush=True)
    rng = np.random.default_rng(rows * 7 + D)
    x = (rng.standard_normal((rows, D)) * 3 + 1).astype(np.float32)
    x[rows // 2, D // 3] = np.float32(250.0)  # one outlier row sets the range
    r = rng.standard_normal((rows, D)).astype(np.float32)
    gam = (rng.standard_normal(D) * 0.5 + 1).astype(np.float32)
    bet = (rng.standard_normal(D) * 0.1).astype(np.float32)
    x1, x2, dr, dg, db = _d(gpu, x), _d(gpu, x), _d(gpu, r), _d(gpu, gam), _d(gpu, bet)
    gp, bp = (dg.data_ptr(), db.data_ptr()) if affine else (None, None)
    y1, y2 = gpu.empty((rows, D), np.float32, "gpu"), gpu.empty((rows, D), np.float32, "gpu")
    q1, q2 = gpu.empty((rows * D,), np.int8, "gpu"), gpu.empty((rows * D + 16,), np.int8, "gpu")
    qp1, qp2 = gpu.empty((4,), np.float32, "gpu"), gpu.empty((4,), np.float32, "gpu")
    eps_ln, eps = np.float32(1e-5), np.float32(1e-8)
    ws_n = _C.lib().lq_dynamic_quantize_workspace_size(rows * D)
    ws = gpu.empty((max(ws_n, 16),), np.uint8, "gpu")
    if with_res:
        _C.call("lq_add_layer_norm_f32", x1.data_ptr(), D, dr.data_ptr(), D, y1.data_ptr(), D, rows, D, gp, bp,
                eps_ln, None)
    else:
        _C.call("lq_layer_norm_f32", x1.data_ptr(), D, y1.data_ptr(), D, rows, D, gp, bp, eps_ln, None)
    _C.call("lq_dynamic_quantize_f32", y1.data_ptr(), rows * D, _C.U8S8, 0, 255, eps, qp1.data_ptr(), q1.data_ptr(),
            ws.data_ptr(), ws_n, None)
    ws2_n = _C.lib().lq_layer_norm_dynamic_quantize_workspace_size(rows, D)
    ws2 = gpu.empty((max(ws2_n, 16),), np.uint8, "gpu")
    _C.call("lq_layer_norm_dynamic_quantize_f32", x2.data_ptr(), D, dr.data_ptr() if with_res else None, D, rows, D,
            gp, bp, eps_ln, y2.data_ptr(), _C.U8S8, 0, 255, eps, qp2.data_ptr(), q2.data_ptr() + qoff, ws2.data_ptr(),
            ws2_n, None)
    n = rows * D
    want_path = ("layer norm dynamic quantize two-launch" if n > 16384 and not qoff
                 else "dynamic quantize fused" if n <= 16384 else "dynamic quantize")
    assert _C.last_path() == want_path
    np.testing.assert_array_equal(x1.numpy().view(np.uint32), x2.numpy().view(np.uint32))
    np.testing.assert_array_equal(y1.numpy().view(np.uint32), y2.numpy().view(np.uint32))
    np.testing.assert_array_equal(q1.numpy(), q2.numpy()[qoff:qoff + n])
    np.testing.assert_array_equal(qp1.numpy().view(np.uint32), qp2.numpy().view(np.uint32))
    # the range came from the data, and the norm matches float64
    want_y = O.layer_norm(x + r if with_res else x, gam if affine else None, bet if affine else None)
    assert_close_to_scale(y2.numpy(), want_y, 1e-5)
    yv = y2.numpy()
    np.testing.assert_array_equal(qp2.numpy()[:2], np.array([yv.min(), yv.max()], np.float32))


def test_layer_norm_quantize_rejects_large(gpu):
    from lucid_amd import _C

    with pytest.raises(_C.LucidError, match="12288"):
        _C.call("lq_layer_norm_quantize_f32", 1, 512, None, 512, 25, 512, None, None, np.float32(1e-5), _C.U8S8, 0,
                255, np.float32(1e-8), 1, 1, None)
