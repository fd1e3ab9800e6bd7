"""GPU parity of HistogramObserver (lq_histc_f32, lq_hist_rebin_f32 and the observer built
on them) against the oracle: bit-exact counts, rebinned histograms, running ranges and
qparams; plus the reference's own unit tests of the observer."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _dev(gpu, a):
    return gpu.tensor(np.ascontiguousarray(a), device="gpu")


def _histc(gpu, x, bins, lo, hi, base=None):
    from lucid_amd import _C

    xt = _dev(gpu, x)
    h = _dev(gpu, base if base is not None else np.zeros(bins, np.float32))
    ws_bytes = _C.lib().lq_histc_workspace_size(bins)
    ws = gpu.empty((ws_bytes,), np.uint8, "gpu")
    _C.call("lq_histc_f32", xt.data_ptr(), x.size, bins, lo, hi, 0 if base is None else 1, h.data_ptr(),
            ws.data_ptr(), ws_bytes, None)
    return h.numpy()


def _edgy(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    idx = rng.choice(n, 64, replace=False)
    x[idx[:8]] = np.nan
    x[idx[8:16]] = np.inf
    x[idx[16:24]] = -np.inf
    return x, rng


@pytest.mark.parametrize("bins", [1, 7, 2048, 20000])
def test_histc_matches_oracle(gpu, bins):
    x, rng = _edgy((1 << 18) + 5, bins)
    finite = x[np.isfinite(x)]
    lo, hi = float(finite.min()) * 0.9, float(finite.max()) * 0.8  # values on both sides too
    x[100:110] = np.float32(lo)   # the bottom edge
    x[200:210] = np.float32(hi)   # the top edge
    np.testing.assert_array_equal(_histc(gpu, x, bins, lo, hi), O.histc(x, bins, lo, hi))
    base = rng.integers(0, 1 << 26, bins).astype(np.float32)   # float32 addition rounds here
    np.testing.assert_array_equal(_histc(gpu, x, bins, lo, hi, base),
                                  (O.histc(x, bins, lo, hi) + base).astype(np.float32))


@pytest.mark.parametrize("ranges", [((-1.0, 2.0), (-3.0, 2.5)), ((0.25, 0.25), (-1.0, 4.0)),
                                    ((-7.5, 1e-3), (-7.5, 31.0)), ((-2.0, 2.0), (-2.0 - 1e-6, 2.0))])
@pytest.mark.parametrize("bins", [2048, 33])
def test_hist_rebin_matches_oracle(gpu, ranges, bins):
    from lucid_amd import _C

    (omin, omax), (nmin, nmax) = ranges
    h = np.random.default_rng(bins).integers(0, 5000, bins).astype(np.float32)
    src = _dev(gpu, h)
    out = gpu.empty((bins,), np.float32, "gpu")
    _C.call("lq_hist_rebin_f32", src.data_ptr(), bins, float(np.float32(omin)),
            float(np.float32((omax - omin) / bins)), float(np.float32(nmin)),
            float(np.float32((nmax - nmin) / bins)), out.data_ptr(), None)
    np.testing.assert_array_equal(out.numpy(), O.hist_rebin(h, omin, omax, nmin, nmax))


def _batches(seed):
    rng = np.random.default_rng(seed)
    b0 = rng.standard_normal(10000).astype(np.float32)
    b1 = (rng.standard_normal(30000) * 4).astype(np.float32)              # widens the range
    b2 = np.clip(rng.standard_normal(5000), -1, 1).astype(np.float32)     # inside: no rebin
    b3 = np.concatenate([rng.standard_normal(777) * 2, [40.0]]).astype(np.float32)  # one side
    return [b0, b1, b2, b3]


@pytest.mark.parametrize("bins", [2048, 512])
def test_observer_matches_oracle(gpu, bins):
    Q = gpu.quantization
    obs = Q.HistogramObserver(bins=bins)
    batches = _batches(bins)
    for k in range(1, len(batches) + 1):
        ys = obs(_dev(gpu, batches[k - 1]))
        mn, mx, hist = O.histogram_observer(batches[:k], bins)
        assert ys.shape == batches[k - 1].shape
        assert obs.min_val.item() == np.float32(mn) and obs.max_val.item() == np.float32(mx)
        np.testing.assert_array_equal(obs.histogram.numpy(), hist)
    cmin, cmax = O.hist_clip_search(hist, mn, mx, 255)
    s_want, z_want = O.calc_qparams(np.float32(cmin), np.float32(cmax), False, False, 0, 255)
    scale, zp = obs.calculate_qparams()
    assert scale.item() == np.float32(s_want) and zp.item() == np.float32(z_want)


def test_observer_constant_first_batch(gpu):
    # a point range counts over [v - 1, v + 1] (the histc adapter), then widens normally
    Q = gpu.quantization
    obs = Q.HistogramObserver(bins=64)
    batches = [np.full(100, 1.5, np.float32), np.linspace(-2, 3, 1000).astype(np.float32)]
    for b in batches:
        obs(_dev(gpu, b))
    mn, mx, hist = O.histogram_observer(batches, 64)
    np.testing.assert_array_equal(obs.histogram.numpy(), hist)
    assert (obs.min_val.item(), obs.max_val.item()) == (np.float32(mn), np.float32(mx))


def test_observer_non_finite(gpu):
    Q = gpu.quantization
    obs = Q.HistogramObserver(bins=32)
    with pytest.raises(ValueError):
        obs(_dev(gpu, np.array([1.0, np.nan, 2.0], np.float32)))
    with pytest.raises(ValueError):
        obs(_dev(gpu, np.array([1.0, np.inf], np.float32)))
    # once a range exists, a NaN batch keeps it (Python min/max skip the NaN extreme) and
    # the NaN elements count nowhere
    obs(_dev(gpu, np.array([0.0, 1.0, 2.0], np.float32)))
    obs(_dev(gpu, np.array([0.5, np.nan], np.float32)))
    assert (obs.min_val.item(), obs.max_val.item()) == (0.0, 2.0)
    assert obs.histogram.numpy().sum() == 4.0


def test_reference_unit_tests(gpu):
    # lucid/test/unit/quantization/test_observer.py:53-76, with numpy's generator
    Q = gpu.quantization
    rng = np.random.default_rng(0)
    obs = Q.HistogramObserver(bins=256)
    obs(_dev(gpu, rng.standard_normal(2000).astype(np.float32)))
    assert obs.histogram.numpy().sum() == pytest.approx(2000, abs=2)
    scale, _ = obs.calculate_qparams()
    assert scale.item() > 0.0
    data = np.concatenate([rng.standard_normal(3000), rng.uniform(5.0, 12.0, 150)]).astype(np.float32)
    h = Q.HistogramObserver(bins=512)
    h(_dev(gpu, data))
    m = Q.MinMaxObserver()
    m(_dev(gpu, data))
    assert h.calculate_qparams()[0].item() <= m.calculate_qparams()[0].item()


def test_default_qconfig_static_flow(gpu):
    # get_default_qconfig (HistogramObserver activations) through prepare / calibrate /
    # convert on a small Linear stack; the converted model runs on the int8 GEMM.
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    rng = np.random.default_rng(5)
    model = nn.Sequential(nnq.QuantStub(), nn.Linear(64, 32), nn.ReLU(), nn.Linear(32, 8),
                          nnq.DeQuantStub()).to("gpu")
    prepared = Q.prepare(model, Q.get_default_qconfig())
    assert isinstance(prepared[1].activation_post_process, Q.HistogramObserver)
    for _ in range(4):
        prepared(_dev(gpu, rng.standard_normal((16, 64)).astype(np.float32)))
    q = Q.convert(prepared)
    y = q(_dev(gpu, rng.standard_normal((16, 64)).astype(np.float32))).numpy()
    assert y.shape == (16, 8) and np.isfinite(y).all()
