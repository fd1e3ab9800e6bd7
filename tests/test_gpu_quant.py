"""GPU parity of the bandwidth kernels (observers, qparams, quantize, dequantize,
fake-quantize) against the CPU oracle and the PyTorch golden fixtures: bit-exact."""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "torch_quant.npz")
SIZES = [1, 15, 16, 17, 1000, 4096 + 3, 1 << 20]


def _data(n, seed=0, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    if outliers and n >= 1000:
        idx = rng.choice(n, max(1, n // 1000), replace=False)
        x[idx] *= 20.0
    return x


def _offset_view(L, arr: np.ndarray, byte_offset: int):
    """A device tensor whose storage starts `byte_offset` bytes into an allocation
    (exercises the unaligned scalar paths)."""
    from lucid_amd._tensor import Tensor, _DeviceBuffer
    from lucid_amd import _C

    t = Tensor()
    t._buf = _DeviceBuffer(arr.nbytes + byte_offset)
    t._offset = byte_offset
    t._shape = arr.shape
    t._dtype = arr.dtype
    t._device = "gpu"
    _C.call("lq_memcpy_h2d", t.data_ptr(), np.ascontiguousarray(arr).ctypes.data, arr.nbytes, None)
    return t


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("case", [("qint8", 0.05, 0), ("qint8", 0.0123, -7), ("quint8", 0.02, 128),
                                  ("qint4", 0.3, 0)])
def test_quantize_per_tensor_python_scale(gpu, n, case):
    Q = gpu.quantization
    name, s, z = case
    qd = getattr(Q, name)
    x = _data(n, seed=n)
    q = Q.quantize(gpu.tensor(x, device="gpu"), s, z, qd).numpy()
    code = O.I16 if qd.storage == "int16" else O.I8
    want = O.quantize(x, O.recip_scalar(s), z, qd.quant_min, qd.quant_max, code)
    assert q.dtype == want.dtype
    np.testing.assert_array_equal(q, want)


@pytest.mark.parametrize("n", SIZES)
def test_quantize_per_tensor_tensor_scale(gpu, n):
    Q = gpu.quantization
    x = _data(n, seed=n + 1)
    s = np.float32(0.0371)
    z = np.float32(5.0)
    q = Q.quantize(gpu.tensor(x, device="gpu"), gpu.tensor(s), gpu.tensor(z), Q.qint8).numpy()
    want = O.quantize(x, O.recip_tensor(s), z, -128, 127, O.I8)
    np.testing.assert_array_equal(q, want)


def test_quantize_unaligned_paths(gpu):
    from lucid_amd import _C

    x = _data(4099, seed=3)
    xt = _offset_view(gpu, x, 4)
    out = _offset_view(gpu, np.zeros(4099, np.int8), 1)
    _C.call("lq_quantize_per_tensor_f32", xt.data_ptr(), out.data_ptr(), x.size, _C.I8, None, None,
            float(O.recip_scalar(0.05)), 0.0, -128, 127, None)
    np.testing.assert_array_equal(out.numpy(), O.quantize(x, O.recip_scalar(0.05), 0, -128, 127))


def test_quantize_edge_values(gpu):
    Q = gpu.quantization
    x = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 0.5, 1.5, 2.5, -2.5, 1e30, -1e30] * 3,
                 np.float32)
    for qd, z in ((Q.qint8, 5.0), (Q.quint8, 0.0), (Q.quint8, 128.0)):
        q = Q.quantize(gpu.tensor(x, device="gpu"), 1.0, z, qd).numpy()
        code = O.I16 if qd.storage == "int16" else O.I8
        np.testing.assert_array_equal(q, O.quantize(x, O.recip_scalar(1.0), z, qd.quant_min,
                                                    qd.quant_max, code))


@pytest.mark.parametrize("code,qmin,qmax,z", [(O.I8, -128, 127, 5.0), (O.U8, 10, 200, 0.5),
                                               (O.U8, 0, 255, 128.0), (O.I16, -128, 127, -3.0),
                                               (O.I32, -1000, 1000, 0.0), (O.U8S8, 0, 255, 128.0),
                                               (O.I8, -300, 300, 0.0)])
def test_quantize_streaming_edges(gpu, code, qmin, qmax, z):
    # The streaming kernel's integer-domain store against the oracle's clip-then-cast, over
    # a tensor large enough to run every block: NaN, infinities, huge values, signed zeros,
    # ties, a grid without 0 (NaN must still store 0), a non-integer zero point and a grid
    # wider than the storage type.
    rng = np.random.default_rng(qmin + qmax + code)
    n = (1 << 20) + 3
    x = (rng.standard_normal(n) * 200).astype(np.float32)
    idx = rng.choice(n, 4000, replace=False)
    x[idx] = rng.choice(np.array([np.nan, np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0, 0.5, -0.5,
                                  2.5, -2.5, 1e9, -1e9], np.float32), 4000)
    from lucid_amd import _C
    npdt = {O.I8: np.int8, O.U8: np.uint8, O.I16: np.int16, O.I32: np.int32, O.U8S8: np.int8}[code]
    xt = gpu.tensor(x, device="gpu")
    out = gpu.tensor(np.zeros(n, npdt), device="gpu")
    inv = float(O.recip_scalar(0.37))
    _C.call("lq_quantize_per_tensor_f32", xt.data_ptr(), out.data_ptr(), n, code, None, None,
            inv, z, qmin, qmax, None)
    np.testing.assert_array_equal(out.numpy(), O.quantize(x, O.recip_scalar(0.37), z, qmin, qmax, code))


@pytest.mark.parametrize("shape,axis", [((48, 64), 0), ((48, 64), 1), ((4096, 256), 0),
                                        ((3, 40, 33), 1), ((64, 256), 1), ((2, 5, 32), 2),
                                        ((256, 784), 0)])
def test_quantize_dequantize_fake_per_channel(gpu, shape, axis):
    Q = gpu.quantization
    rng = np.random.default_rng(sum(shape) + axis)
    x = rng.standard_normal(shape).astype(np.float32) * 2
    C = shape[axis]
    s = rng.uniform(0.005, 0.05, C).astype(np.float32)
    z = rng.integers(-3, 4, C).astype(np.float32)
    xd = gpu.tensor(x, device="gpu")
    q = Q.quantize(xd, gpu.tensor(s), gpu.tensor(z), Q.qint8, ch_axis=axis)
    want = O.quantize(x, O.recip_tensor(s), z, -128, 127, O.I8, ch_axis=axis)
    np.testing.assert_array_equal(q.numpy(), want)
    dq = Q.dequantize(q, gpu.tensor(s), gpu.tensor(z), ch_axis=axis).numpy()
    np.testing.assert_array_equal(dq, O.dequantize(want, O.I8, s, z, ch_axis=axis))
    dh = Q.dequantize(q, gpu.tensor(s), gpu.tensor(z), ch_axis=axis, out_dtype=gpu.float16).numpy()
    np.testing.assert_array_equal(dh.view(np.uint16),
                                  O.dequantize(want, O.I8, s, z, ch_axis=axis, y_dtype=O.F16)
                                  .view(np.uint16))
    fq, mask = Q.fake_quantize(xd, gpu.tensor(s), gpu.tensor(z), -128, 127, ch_axis=axis,
                               return_mask=True)
    wfq, wmask = O.fake_quantize(x, O.recip_tensor(s), s, z, -128, 127, ch_axis=axis)
    np.testing.assert_array_equal(fq.numpy(), wfq)
    np.testing.assert_array_equal(mask.numpy(), wmask)


@pytest.mark.parametrize("n", SIZES)
def test_dequantize_and_fake_per_tensor(gpu, n):
    Q = gpu.quantization
    x = _data(n, seed=n + 2)
    for qd, s, z in ((Q.qint8, 0.05, 3), (Q.quint8, 0.031, 128)):
        code = O.I16 if qd.storage == "int16" else O.I8
        q = O.quantize(x, O.recip_scalar(s), z, qd.quant_min, qd.quant_max, code)
        qt = gpu.tensor(q, device="gpu")
        np.testing.assert_array_equal(Q.dequantize(qt, s, z).numpy(),
                                      O.dequantize(q, code, np.float32(s), z))
        h = Q.dequantize(qt, s, z, out_dtype=gpu.float16).numpy()
        np.testing.assert_array_equal(h.view(np.uint16),
                                      O.dequantize(q, code, np.float32(s), z, y_dtype=O.F16)
                                      .view(np.uint16))
        fq, m = Q.fake_quantize(gpu.tensor(x, device="gpu"), s, z, qd.quant_min, qd.quant_max,
                                return_mask=True)
        wfq, wm = O.fake_quantize(x, O.recip_scalar(s), np.float32(s), z, qd.quant_min,
                                  qd.quant_max)
        np.testing.assert_array_equal(fq.numpy(), wfq)
        np.testing.assert_array_equal(m.numpy(), wm)


def test_torch_golden_fixtures(gpu):
    Q = gpu.quantization
    g = np.load(GOLDEN)
    x = gpu.tensor(g["pt_x"], device="gpu")
    for i, (s, z, signed) in enumerate(zip(g["pt_scale"], g["pt_zp"], g["pt_signed"])):
        qd = Q.qint8 if signed else Q.quint8
        q = Q.quantize(x, float(s), int(z), qd)
        np.testing.assert_array_equal(q.numpy().astype(np.int16), g["pt_codes"][i])
        np.testing.assert_array_equal(Q.dequantize(q, float(s), int(z)).numpy(), g["pt_dequant"][i])
        np.testing.assert_array_equal(
            Q.fake_quantize(x, float(s), int(z), qd.quant_min, qd.quant_max).numpy(), g["pt_fake"][i])
    w = gpu.tensor(g["pc_w"], device="gpu")
    for ax in (0, 1):
        sc = gpu.tensor(g[f"pc{ax}_scale"])
        zp = gpu.tensor(np.zeros(g["pc_w"].shape[ax], np.float32))
        np.testing.assert_array_equal(Q.quantize(w, sc, zp, Q.qint8, ch_axis=ax).numpy(),
                                      g[f"pc{ax}_codes"])
        np.testing.assert_array_equal(Q.fake_quantize(w, sc, zp, -128, 127, ch_axis=ax).numpy(),
                                      g[f"pc{ax}_fake"])


# ------------------------------------------------------------------ observers


@pytest.mark.parametrize("n", [0, 1, 3, 1000, 4096 + 3, 1 << 20, (1 << 22) + 5])
def test_minmax_observer(gpu, n):
    Q = gpu.quantization
    obs = Q.MinMaxObserver()
    ema = Q.MovingAverageMinMaxObserver(averaging_constant=0.1)
    r = np.array([np.inf, -np.inf], np.float32)
    e = r.copy()
    for k in range(3):
        x = _data(n, seed=100 + k) * (k + 1)
        xd = gpu.tensor(x, device="gpu")
        obs(xd)
        ema(xd)
        r = O.minmax(x, r)
        e = O.minmax(x, e, mode=O.OBS_EMA, c=0.1)
    np.testing.assert_array_equal([obs.min_val.item(), obs.max_val.item()], r)
    np.testing.assert_array_equal([ema.min_val.item(), ema.max_val.item()], e)
    s, z = obs.calculate_qparams()
    ws, wz = O.calc_qparams(r[0], r[1], False, False, 0, 255)
    assert s.item() == ws.item() and z.item() == wz.item()


def test_minmax_nan_and_signed_zero(gpu):
    Q = gpu.quantization
    x = _data(50000, seed=7)
    x[12345] = np.nan
    obs = Q.MinMaxObserver()
    obs(gpu.tensor(x, device="gpu"))
    assert np.isnan(obs.min_val.item()) and np.isnan(obs.max_val.item())
    neg_nan = np.array([1.0, -np.nan, 2.0], np.float32)
    obs = Q.MinMaxObserver()
    obs(gpu.tensor(neg_nan, device="gpu"))
    assert np.isnan(obs.min_val.item()) and np.isnan(obs.max_val.item())
    z = np.array([0.0, -0.0, 0.0], np.float32)
    obs = Q.MinMaxObserver()
    obs(gpu.tensor(z, device="gpu"))
    assert np.signbit(obs.min_val.item()) and not np.signbit(obs.max_val.item())


@pytest.mark.parametrize("shape,axis", [((6, 10), 0), ((64, 256), 1), ((4096, 300), 0),
                                        ((3, 40, 33), 1), ((8, 4, 100), 2), ((16, 3, 5, 5), 0),
                                        ((256, 784), 0), ((10, 256), 0), ((2, 0, 3), 0)])
def test_per_channel_observers(gpu, shape, axis):
    Q = gpu.quantization
    pc = Q.PerChannelMinMaxObserver(ch_axis=axis)
    ema = Q.MovingAveragePerChannelMinMaxObserver(ch_axis=axis, averaging_constant=0.1)
    rmin = rmax = emin = emax = None
    for k in range(2):
        x = np.random.default_rng(k + sum(shape)).standard_normal(shape).astype(np.float32)
        xd = gpu.tensor(x, device="gpu")
        pc(xd)
        ema(xd)
        rmin, rmax = O.minmax_per_channel(x, axis, rmin, rmax)
        emin, emax = O.minmax_per_channel(x, axis, emin, emax, mode=O.OBS_EMA, c=0.1)
    np.testing.assert_array_equal(pc.min_val.numpy(), rmin)
    np.testing.assert_array_equal(pc.max_val.numpy(), rmax)
    np.testing.assert_array_equal(ema.min_val.numpy(), emin)
    np.testing.assert_array_equal(ema.max_val.numpy(), emax)
    if shape[axis]:
        s, z = pc.calculate_qparams()
        ws, wz = O.calc_qparams(rmin, rmax, True, True, -128, 127)
        np.testing.assert_array_equal(s.numpy(), ws)
        np.testing.assert_array_equal(z.numpy(), wz)


def test_calculate_qparams_grid(gpu):
    Q = gpu.quantization
    rng = np.random.default_rng(11)
    mn = np.concatenate([-rng.exponential(2, 500), [0.0, -0.0, np.inf, -np.inf, np.nan, -1e-12,
                                                     -3.0]]).astype(np.float32)
    mx = np.concatenate([rng.exponential(2, 500), [0.0, 0.0, -np.inf, np.inf, 1.0, 1e-12,
                                                   -1.0]]).astype(np.float32)
    for scheme in (Q.per_tensor_affine, Q.per_tensor_symmetric):
        for qd in (Q.qint8, Q.quint8, Q.qint4):
            s, z = Q.calculate_qparams(gpu.tensor(mn), gpu.tensor(mx), scheme, qd)
            ws, wz = O.calc_qparams(mn, mx, scheme.is_symmetric, qd.signed, qd.quant_min,
                                    qd.quant_max)
            np.testing.assert_array_equal(s.numpy(), ws)
            np.testing.assert_array_equal(z.numpy(), wz)


def test_observer_state_dict_round_trip(gpu):
    Q = gpu.quantization
    obs = Q.MinMaxObserver()
    obs(gpu.tensor(np.array([-2.0, 5.0], np.float32), device="gpu"))
    sd = obs.state_dict()
    assert list(sd) == ["min_val", "max_val"]
    assert sd["min_val"].shape == () and sd["max_val"].shape == ()
    fresh = Q.MinMaxObserver()
    fresh.load_state_dict(sd)
    assert fresh.min_val.item() == -2.0 and fresh.max_val.item() == 5.0
    pc = Q.PerChannelMinMaxObserver(ch_axis=0)
    pc(gpu.tensor(np.arange(12, dtype=np.float32).reshape(4, 3), device="gpu"))
    fresh = Q.PerChannelMinMaxObserver(ch_axis=0)
    fresh.load_state_dict(pc.state_dict())
    np.testing.assert_array_equal(fresh.min_val.numpy(), [0, 3, 6, 9])


# ------------------------------------------------------ dynamic activation quantization


def _dyn_inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    if n > 8:
        x[3] = np.float32(-0.0)
        x[n // 2] *= np.float32(40.0)  # an outlier sets the range
    return x


_DYN_CASES = [(n, 0) for n in (1, 5, 4096, 4097, 16384, 16385, 300000, 8 * 2**20 + 3)] + [(16385, 1), (300000, 1)]


@pytest.mark.parametrize("n,offset", _DYN_CASES)
@pytest.mark.parametrize("grid", [(0, 255, "U8S8"), (-128, 127, "I8")])
def test_dynamic_quantize_matches_separate_calls(gpu, n, grid, offset):
    """lq_dynamic_quantize_f32 (one launch up to 16384 elements; above, two launches when the
    float and code vectors are aligned -- offset 0 -- else the separate launches: offset 1
    starts the input one float past alignment) against the
    observer -> qparams -> quantize launches it replaces, and against the oracle: the min, max,
    scale, zero point and every code the same bits.  8 Mi + 3 elements folds the largest
    number of extrema partials and quantizes a tail past the last group of four."""
    from lucid_amd import _C

    qmin, qmax, ct = grid
    code_type = getattr(_C, ct)
    x = _dyn_inputs(n, n + abs(qmin))
    xbuf = gpu.tensor(np.concatenate([np.zeros(offset, np.float32), x]), device="gpu")
    xp = xbuf.data_ptr() + 4 * offset
    eps = float(np.float32(1e-8))
    qp = gpu.empty((4,), np.float32, "gpu")
    codes = gpu.empty((n,), np.int8, "gpu")
    ws_bytes = _C.lib().lq_dynamic_quantize_workspace_size(n)
    ws = gpu.empty((max(ws_bytes, 16),), np.uint8, "gpu")
    _C.call("lq_dynamic_quantize_f32", xp, n, code_type, qmin, qmax, eps, qp.data_ptr(),
            codes.data_ptr(), ws.data_ptr(), ws_bytes, None)
    gpu.synchronize()
    want_path = ("dynamic quantize fused" if n <= 16384
                 else "dynamic quantize" if offset else "dynamic quantize two-launch")
    assert _C.last_path() == want_path
    # the separate launches
    qp2 = gpu.empty((4,), np.float32, "gpu")
    codes2 = gpu.empty((n,), np.int8, "gpu")
    mm_bytes = _C.lib().lq_minmax_workspace_size(n)
    mm = gpu.empty((mm_bytes,), np.uint8, "gpu")
    p = qp2.data_ptr()
    _C.call("lq_minmax_f32", xp, n, p, p + 4, _C.OBS_REPLACE, 0.0, mm.data_ptr(), mm_bytes, None)
    _C.call("lq_calc_qparams_f32", p, p + 4, 1, 0, int(qmin < 0), qmin, qmax, eps, p + 8, p + 12, None)
    _C.call("lq_quantize_per_tensor_f32", xp, codes2.data_ptr(), n, code_type, p + 8, p + 12, 0.0, 0.0,
            qmin, qmax, None)
    a, b = qp.numpy(), qp2.numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    np.testing.assert_array_equal(codes.numpy(), codes2.numpy())
    # the oracle
    mn, mx = O.minmax(x, mode=O.OBS_REPLACE)
    s, z = O.calc_qparams(mn, mx, False, qmin < 0, qmin, qmax)
    want = O.quantize(x, O.recip_tensor(np.array([s], np.float32))[0], z, qmin, qmax,
                      O.U8S8 if ct == "U8S8" else O.I8)
    np.testing.assert_array_equal(a.view(np.uint32), np.array([mn, mx, s, z], np.float32).view(np.uint32))
    np.testing.assert_array_equal(codes.numpy(), want.astype(np.int8))


def test_dynamic_quantize_empty_input(gpu):
    """n = 0 runs the separate launches (no element is read or written; the two-launch form's
    read-ahead needs at least one group) and returns without error, as before the two-launch
    form existed."""
    from lucid_amd import _C

    qp = gpu.empty((4,), np.float32, "gpu")
    ws_n = _C.lib().lq_dynamic_quantize_workspace_size(0)
    ws = gpu.empty((max(ws_n, 16),), np.uint8, "gpu")
    _C.call("lq_dynamic_quantize_f32", None, 0, _C.U8S8, 0, 255, np.float32(1e-8), qp.data_ptr(), None,
            ws.data_ptr(), ws_n, None)
    gpu.synchronize()
    assert _C.last_path() == "dynamic quantize"


def test_dynamic_quantize_edge_ranges(gpu):
    """Zero range (all equal), negative-only, NaN and infinities: the fused launches against the
    separate ones, at one-launch sizes and (tiled past 16384 elements) two-launch sizes."""
    from lucid_amd import _C

    eps = float(np.float32(1e-8))
    cases = [np.full(100, 1.5, np.float32), -np.abs(_dyn_inputs(777, 1)), np.zeros(64, np.float32),
             np.array([1.0, np.nan, -2.0, 3.0] * 50, np.float32), np.array([np.inf, -1.0, 2.0] * 30, np.float32)]
    cases += [np.tile(c, 70000 // c.size + 1) for c in cases]
    for x in cases:
        n = x.size
        xd = gpu.tensor(x, device="gpu")
        out = []
        for fused in (True, False):
            qp = gpu.empty((4,), np.float32, "gpu")
            codes = gpu.empty((n,), np.int8, "gpu")
            if fused:
                ws_bytes = _C.lib().lq_dynamic_quantize_workspace_size(n)
                ws = gpu.empty((max(ws_bytes, 16),), np.uint8, "gpu")
                _C.call("lq_dynamic_quantize_f32", xd.data_ptr(), n, _C.U8S8, 0, 255, eps, qp.data_ptr(),
                        codes.data_ptr(), ws.data_ptr() if ws_bytes else None, ws_bytes, None)
                assert _C.last_path() == ("dynamic quantize fused" if n <= 16384 else "dynamic quantize two-launch")
            else:
                mm_bytes = _C.lib().lq_minmax_workspace_size(n)
                mm = gpu.empty((mm_bytes,), np.uint8, "gpu")
                p = qp.data_ptr()
                _C.call("lq_minmax_f32", xd.data_ptr(), n, p, p + 4, _C.OBS_REPLACE, 0.0, mm.data_ptr(), mm_bytes,
                        None)
                _C.call("lq_calc_qparams_f32", p, p + 4, 1, 0, 0, 0, 255, eps, p + 8, p + 12, None)
                _C.call("lq_quantize_per_tensor_f32", xd.data_ptr(), codes.data_ptr(), n, _C.U8S8, p + 8, p + 12,
                        0.0, 0.0, 0, 255, None)
            out.append((qp.numpy(), codes.numpy()))
        np.testing.assert_array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
        np.testing.assert_array_equal(out[0][1], out[1][1])
