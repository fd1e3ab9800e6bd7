"""GPU parity of the table lookups (lq_embedding / lq_embedding_bag, nn.Embedding /
nn.EmbeddingBag and the int8 nn.quantized.Embedding / EmbeddingBag) against the oracle.

The quantized lookup dequantizes only the rows it reads; its result must equal the oracle's
lookup over the table dequantized as Lucid does it (dequantize(..., ch_axis=0), then the
float lookup): bit-exact for every mode, bag layout, padding index and per-sample weight,
on the 4-wide and the 1-wide paths.  Plus the reference's module test
(lucid/test/unit/quantization/test_module_breadth.py:92-105) and the index rules.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _dev(gpu, a):
    return gpu.tensor(np.ascontiguousarray(a), device="gpu")


def _int8_table(rng, rows, D):
    w = (rng.standard_normal((rows, D)) * rng.uniform(0.1, 3.0, (rows, 1))).astype(np.float32)
    s = (np.abs(w).max(1) / 127.5 + 1e-8).astype(np.float32)
    z = rng.integers(-3, 4, rows).astype(np.float32)
    codes = O.quantize(w, O.recip_tensor(s), z, -128, 127, O.I8, ch_axis=0)
    return codes, s, z, O.dequantize(codes, O.I8, s, z, ch_axis=0)


def _bag(gpu, codes, s, z, idx, offsets=None, mode=O.BAG_MEAN, pad=-1, last=False, bag_len=0, psw=None,
         idx_dtype=np.int64, float_table=None):
    from lucid_amd import _C

    rows, D = (float_table if float_table is not None else codes).shape
    n_bags = (len(offsets) - (1 if last else 0)) if offsets is not None else idx.size // bag_len
    t = _dev(gpu, float_table if float_table is not None else codes)
    sd, zd = (None, None) if float_table is not None else (_dev(gpu, s), _dev(gpu, z))
    it = _dev(gpu, idx.astype(idx_dtype))
    ot = _dev(gpu, np.asarray(offsets, np.int32)) if offsets is not None else None
    wd = _dev(gpu, psw.astype(np.float32)) if psw is not None else None
    y = gpu.empty((n_bags, D), np.float32, "gpu")
    _C.call("lq_embedding_bag", t.data_ptr(), _C.F32 if float_table is not None else _C.I8,
            sd.data_ptr() if sd is not None else None, zd.data_ptr() if zd is not None else None, rows, D,
            it.data_ptr(), _C.I64 if idx_dtype == np.int64 else _C.I32, idx.size,
            ot.data_ptr() if ot is not None else None, _C.I32, len(offsets) if offsets is not None else 0,
            1 if last else 0, bag_len, mode, pad, wd.data_ptr() if wd is not None else None, y.data_ptr(), None)
    return y.numpy()


@pytest.mark.parametrize("D", [1, 3, 16, 64, 100, 512])
@pytest.mark.parametrize("idx_dtype", [np.int32, np.int64])
def test_embedding_lookup_exact(gpu, D, idx_dtype):
    from lucid_amd import _C

    rng = np.random.default_rng(D)
    rows = 1000
    codes, s, z, deq = _int8_table(rng, rows, D)
    idx = rng.integers(0, rows, (7, 33)).astype(idx_dtype)
    out = gpu.empty((idx.size, D), np.float32, "gpu")
    t, sd, zd, it = _dev(gpu, codes), _dev(gpu, s), _dev(gpu, z), _dev(gpu, idx)
    _C.call("lq_embedding", t.data_ptr(), _C.I8, sd.data_ptr(), zd.data_ptr(), rows, D, it.data_ptr(),
            _C.I64 if idx_dtype == np.int64 else _C.I32, idx.size, out.data_ptr(), None)
    np.testing.assert_array_equal(out.numpy(), deq[idx.ravel()])
    # the float table through the same kernel
    ft = _dev(gpu, deq)
    _C.call("lq_embedding", ft.data_ptr(), _C.F32, None, None, rows, D, it.data_ptr(),
            _C.I64 if idx_dtype == np.int64 else _C.I32, idx.size, out.data_ptr(), None)
    np.testing.assert_array_equal(out.numpy(), deq[idx.ravel()])


@pytest.mark.parametrize("mode", [O.BAG_SUM, O.BAG_MEAN, O.BAG_MAX])
@pytest.mark.parametrize("D", [4, 7, 128])
@pytest.mark.parametrize("layout", ["offsets", "last_offset", "2d"])
def test_embedding_bag_exact(gpu, mode, D, layout):
    rng = np.random.default_rng(mode * 100 + D + len(layout))
    rows = 500
    codes, s, z, deq = _int8_table(rng, rows, D)
    n = 300
    idx = rng.integers(0, rows, n)
    pad = int(idx[5])
    if layout == "2d":
        kw = dict(bag_len=20)
        ref = O.embedding_bag(deq, idx, None, mode, padding_idx=pad, bag_len=20)
        got = _bag(gpu, codes, s, z, idx, None, mode, pad, bag_len=20)
    else:
        offsets = np.sort(rng.integers(0, n + 1, 40))
        offsets[0] = 0
        offsets[7] = offsets[8] = offsets[6]  # empty bags
        last = layout == "last_offset"
        ref = O.embedding_bag(deq, idx, offsets, mode, padding_idx=pad, include_last_offset=last)
        got = _bag(gpu, codes, s, z, idx, offsets, mode, pad, last=last)
    np.testing.assert_array_equal(got, ref)


def test_embedding_bag_per_sample_weights_and_float_table(gpu):
    rng = np.random.default_rng(3)
    rows, D = 200, 24
    codes, s, z, deq = _int8_table(rng, rows, D)
    idx = rng.integers(0, rows, 150)
    offsets = np.array([0, 10, 10, 77, 120])
    w = rng.standard_normal(150).astype(np.float32)
    pad = int(idx[12])
    ref = O.embedding_bag(deq, idx, offsets, O.BAG_SUM, padding_idx=pad, per_sample_weights=w)
    np.testing.assert_array_equal(_bag(gpu, codes, s, z, idx, offsets, O.BAG_SUM, pad, psw=w), ref)
    table = (rng.standard_normal((rows, D)) * 5).astype(np.float32)
    ref = O.embedding_bag(table, idx, offsets, O.BAG_MEAN, padding_idx=pad)
    np.testing.assert_array_equal(_bag(gpu, None, None, None, idx, offsets, O.BAG_MEAN, pad, float_table=table,
                                       idx_dtype=np.int32), ref)


def test_bad_index_reads_nan(gpu):
    # the reference's GPU policy: an out-of-range index is isolated as NaN, not read
    rng = np.random.default_rng(8)
    codes, s, z, deq = _int8_table(rng, 10, 8)
    idx = np.array([1, 2, 10, 3, -1, 4])
    got = _bag(gpu, codes, s, z, idx, np.array([0, 2, 4]), O.BAG_SUM)
    np.testing.assert_array_equal(got[0], O.embedding_bag(deq, idx[:2], np.array([0]), O.BAG_SUM)[0])
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()


def test_quantized_embedding_bag_module(gpu):
    # lucid/test/unit/quantization/test_module_breadth.py:92-105
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq
    from lucid_amd.nn.layers import manual_seed

    Q = gpu.quantization
    manual_seed(0)
    m = nn.Sequential(nn.EmbeddingBag(50, 16, mode="mean")).to("gpu")
    idx = _dev(gpu, np.array([1, 5, 9, 3, 7, 2, 8], np.int64))
    off = _dev(gpu, np.array([0, 3, 5], np.int64))
    yf = m[0](idx, off).numpy()
    np.testing.assert_array_equal(yf, O.embedding_bag(m[0].weight.numpy(), idx.numpy(), off.numpy(), O.BAG_MEAN))
    qm = Q.convert(m)
    assert isinstance(qm[0], nnq.EmbeddingBag)
    assert qm[0].weight_int8.dtype == np.int8
    yq = qm[0](idx, off).numpy()
    assert np.abs(yf - yq).max() / (np.abs(yf).max() + 1e-9) < 0.05
    deq = O.dequantize(qm[0].weight_int8.numpy(), O.I8, qm[0].weight_scale.numpy(),
                       qm[0].weight_zero_point.numpy(), ch_axis=0)
    np.testing.assert_array_equal(yq, O.embedding_bag(deq, idx.numpy(), off.numpy(), O.BAG_MEAN))
    assert list(qm.state_dict()) == ["0.weight_int8", "0.weight_scale", "0.weight_zero_point"]


def test_quantized_embedding_module_and_index_rules(gpu, monkeypatch):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    Q = gpu.quantization
    m = nn.Sequential(nn.Embedding(40, 12, padding_idx=-1)).to("gpu")
    assert m[0].padding_idx == 39 and not m[0].weight.numpy()[39].any()
    idx = np.array([[0, 39, 5], [7, 7, 38]], np.int64)
    q = Q.convert(m)[0]
    assert isinstance(q, nnq.Embedding) and q.padding_idx == 39
    y = q(_dev(gpu, idx))
    assert y.shape == (2, 3, 12)
    deq = O.dequantize(q.weight_int8.numpy(), O.I8, q.weight_scale.numpy(), q.weight_zero_point.numpy(),
                       ch_axis=0)
    np.testing.assert_array_equal(y.numpy(), deq[idx])
    with pytest.raises(TypeError):
        q(_dev(gpu, idx.astype(np.float32)))
    monkeypatch.setenv("LUCID_STRICT_INDEX", "1")
    with pytest.raises(IndexError):
        q(_dev(gpu, np.array([0, 40])))
    bag = nnq.EmbeddingBag.from_float(nn.EmbeddingBag(40, 12).to("gpu"))
    with pytest.raises(ValueError):
        bag(_dev(gpu, np.array([1, 2, 3])), _dev(gpu, np.array([1, 2])))   # offsets[0] != 0
    with pytest.raises(IndexError):
        bag(_dev(gpu, np.array([1, 2, 3])), _dev(gpu, np.array([0, 4])))   # past the indices
    with pytest.raises(ValueError):
        bag(_dev(gpu, np.array([1, 2, 3])), _dev(gpu, np.array([0, 2, 1])))  # decreasing
    with pytest.raises(NotImplementedError):
        bag(_dev(gpu, np.array([1, 2, 3])), _dev(gpu, np.array([0])), _dev(gpu, np.ones(3, np.float32)))


@pytest.mark.parametrize("bag", [False, True])
def test_qpair_table_matches_separate_qparams(gpu, bag):
    """LQ_I8_QPAIR (one interleaved {scale, zero point} pair per row) against LQ_I8 with separate
    scale / zero-point arrays: the same dequantization, bit for bit."""
    from lucid_amd import _C

    rng = np.random.default_rng(7 + bag)
    rows, D = 300, 40
    codes = rng.integers(-128, 128, (rows, D)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-1, rows).astype(np.float32)
    z = rng.integers(-20, 21, rows).astype(np.float32)
    idx = rng.integers(0, rows, 64).astype(np.int64)
    idx[5] = rows + 3  # out of range: NaN either way
    t, sd, zd, pd = (gpu.tensor(a, device="gpu") for a in (codes, s, z, np.stack([s, z], 1)))
    ii = gpu.tensor(idx, device="gpu")
    outs = []
    for tt, sp, zp in ((_C.I8, sd.data_ptr(), zd.data_ptr()), (_C.I8_QPAIR, pd.data_ptr(), None)):
        if bag:
            y = gpu.empty((16, D), np.float32, "gpu")
            _C.call("lq_embedding_bag", t.data_ptr(), tt, sp, zp, rows, D, ii.data_ptr(), _C.I64, 64, None,
                    _C.I64, 0, 0, 4, _C.BAG_MEAN, -1, None, y.data_ptr(), None)
        else:
            y = gpu.empty((64, D), np.float32, "gpu")
            _C.call("lq_embedding", t.data_ptr(), tt, sp, zp, rows, D, ii.data_ptr(), _C.I64, 64, y.data_ptr(), None)
        outs.append(y.numpy())
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.isnan(outs[1]).any()


def test_quantized_table_follows_in_place_state_dict_loads(gpu):
    """load_state_dict copies into the module's buffers in place: the next lookup must use the
    new scales / zero points (a module that cached anything derived from them would not)."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    rng = np.random.default_rng(3)
    src = nn.EmbeddingBag(50, 16, mode="sum")
    src.weight = nn.Parameter(gpu.tensor(rng.standard_normal((50, 16)).astype(np.float32)))
    q = nnq.EmbeddingBag.from_float(src)
    idx = gpu.tensor(rng.integers(0, 50, (4, 3)).astype(np.int64), device="gpu")
    first = q(idx).numpy()
    sd = q.state_dict()
    sd2 = {k: (gpu.tensor(v.numpy() * 2) if k.endswith("weight_scale") else v) for k, v in sd.items()}
    q.load_state_dict(sd2)
    np.testing.assert_allclose(q(idx).numpy(), 2 * first, rtol=1e-6, atol=1e-6)
