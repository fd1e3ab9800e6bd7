"""GPU parity of the recurrent layers (lq_rnn_cell inside nn.LSTM / GRU / LSTMCell / GRUCell /
RNNCell and their dynamic int8 forms in nn.quantized.dynamic) against the oracle's float64
recurrence.

* float modules: the oracle over the same float32 weights; float32 products and gate math
  against float64, absolute tolerance 2e-5 (states are bounded by tanh / sigmoid);
* dynamic modules: the oracle over the dequantized weights (Lucid's forward: dequantize, then
  the float module, lucid/nn/quantized/dynamic/rnn.py:35-56), same tolerance, the weight codes
  and scales bit-exact against the oracle's per-channel symmetric quantization;
* the reference's own tests (lucid/test/unit/quantization/test_dynamic_recurrent.py:44-150):
  every type converts, holds int8 codes and no float weight, stays within 3% of the float
  module, and leaves the float module alone.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ATOL = 2e-5


def _dev(gpu, a):
    return gpu.tensor(np.ascontiguousarray(a, dtype=np.float32), device="gpu")


def _float_weights(mod):
    return {n: p.numpy().astype(np.float64) for n, p in mod.named_parameters()}


def _deq_weights(q):
    out = {}
    for n, b in q.named_buffers():
        if n.endswith("_int8"):
            out[n[:-5]] = b.numpy().astype(np.float64) * q._buffers[n[:-5] + "_scale"].numpy().astype(np.float64)[:, None]
        elif not n.endswith("_scale"):
            out[n] = b.numpy().astype(np.float64)
    return out


MODES = [("LSTM", 1, False, False), ("LSTM", 2, True, False), ("GRU", 1, False, True), ("GRU", 2, True, True)]


@pytest.mark.parametrize("mode,layers,bidir,batch_first", MODES)
def test_sequence_modules_match_oracle(gpu, mode, layers, bidir, batch_first):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.nn.layers import manual_seed

    manual_seed(layers + 3 * bidir)
    rng = np.random.default_rng(layers)
    T, B, I, H = 7, 3, 10, 16
    m = getattr(nn, mode)(I, H, num_layers=layers, bidirectional=bidir, batch_first=batch_first).to("gpu")
    x = rng.standard_normal((T, B, I)).astype(np.float32)
    D = 2 if bidir else 1
    h0 = (rng.standard_normal((layers * D, B, H)) * 0.5).astype(np.float32)
    c0 = (rng.standard_normal((layers * D, B, H)) * 0.5).astype(np.float32)
    xin = x.transpose(1, 0, 2) if batch_first else x
    hx = (_dev(gpu, h0), _dev(gpu, c0)) if mode == "LSTM" else _dev(gpu, h0)
    for mod, weights in ((m, _float_weights(m)), (None, None)):
        if mod is None:
            mod = nnqd.__dict__[mode].from_float(m)
            weights = _deq_weights(mod)
        out, state = mod(_dev(gpu, xin), hx)
        want, h_n, c_n = O.rnn_forward(mode, x, weights, layers, bidir, h0, c0 if mode == "LSTM" else None)
        got = out.numpy().transpose(1, 0, 2) if batch_first else out.numpy()
        np.testing.assert_allclose(got, want, atol=ATOL, rtol=0)
        if mode == "LSTM":
            np.testing.assert_allclose(state[0].numpy(), h_n, atol=ATOL, rtol=0)
            np.testing.assert_allclose(state[1].numpy(), c_n, atol=ATOL, rtol=0)
        else:
            np.testing.assert_allclose(state.numpy(), h_n, atol=ATOL, rtol=0)


@pytest.mark.parametrize("cell,mode", [("LSTMCell", "LSTM"), ("GRUCell", "GRU"), ("RNNCell", "RNN_TANH"),
                                       ("RNNCell-relu", "RNN_RELU")])
def test_cells_match_oracle(gpu, cell, mode):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd

    rng = np.random.default_rng(len(cell))
    B, I, H = 5, 12, 9
    name = cell.split("-")[0]
    m = (nn.RNNCell(I, H, nonlinearity="relu") if cell.endswith("relu") else getattr(nn, name)(I, H)).to("gpu")
    x = rng.standard_normal((B, I)).astype(np.float32)
    h = (rng.standard_normal((B, H)) * 0.5).astype(np.float32)
    c = (rng.standard_normal((B, H)) * 0.5).astype(np.float32)
    for mod in (m, nnqd.__dict__[name].from_float(m)):
        w = _float_weights(mod) if mod is m else _deq_weights(mod)
        hx = (_dev(gpu, h), _dev(gpu, c)) if mode == "LSTM" else _dev(gpu, h)
        res = mod(_dev(gpu, x), hx)
        gx = x.astype(np.float64) @ w["weight_ih"].T + w["bias_ih"]
        gh = h.astype(np.float64) @ w["weight_hh"].T + w["bias_hh"]
        want_h, want_c = O.rnn_cell(mode, gx, gh, h.astype(np.float64), c.astype(np.float64))
        got_h = res[0] if mode == "LSTM" else res
        np.testing.assert_allclose(got_h.numpy(), want_h, atol=ATOL, rtol=0)
        if mode == "LSTM":
            np.testing.assert_allclose(res[1].numpy(), want_c, atol=ATOL, rtol=0)


def test_dynamic_weights_are_the_oracle_codes(gpu):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd

    m = nn.GRU(6, 8, num_layers=2, bidirectional=True).to("gpu")
    q = nnqd.GRU.from_float(m)
    for name, p in m.named_parameters():
        if not name.startswith("weight"):
            np.testing.assert_array_equal(q._buffers[name].numpy(), p.numpy())
            continue
        W = p.numpy()
        mn, mx = O.minmax_per_channel(W, 0)
        s, z = O.calc_qparams(mn, mx, True, True, -128, 127)
        np.testing.assert_array_equal(q._buffers[name + "_scale"].numpy(), s)
        np.testing.assert_array_equal(q._buffers[name + "_int8"].numpy(),
                                      O.quantize(W, O.recip_tensor(s), z, -128, 127, O.I8, ch_axis=0))


_CASES = {
    "Linear": (lambda nn: nn.Linear(4, 6), (3, 4)),
    "LSTM": (lambda nn: nn.LSTM(4, 6, num_layers=2), (5, 2, 4)),
    "GRU": (lambda nn: nn.GRU(4, 6), (5, 2, 4)),
    "GRU-2layer-bidir": (lambda nn: nn.GRU(4, 6, num_layers=2, bidirectional=True), (5, 2, 4)),
    "LSTMCell": (lambda nn: nn.LSTMCell(4, 6), (3, 4)),
    "GRUCell": (lambda nn: nn.GRUCell(4, 6), (3, 4)),
    "RNNCell-tanh": (lambda nn: nn.RNNCell(4, 6), (3, 4)),
    "RNNCell-relu": (lambda nn: nn.RNNCell(4, 6, nonlinearity="relu"), (3, 4)),
}


@pytest.fixture()
def reference_engine():
    import lucid_amd.backends as backends

    backends.quantized.engine = "reference"
    yield
    backends.quantized.engine = "auto"


@pytest.mark.parametrize("case", list(_CASES))
def test_each_type_is_quantized_and_stays_close(gpu, reference_engine, case):
    # lucid/test/unit/quantization/test_dynamic_recurrent.py:78-100
    import warnings

    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.nn.layers import manual_seed
    from lucid_amd.quantization import quantize_dynamic

    make, shape = _CASES[case]
    manual_seed(0)
    model = nn.Sequential(make(nn)).to("gpu")
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        qmodel = quantize_dynamic(model)
    qtype = getattr(nnqd, case.split("-")[0])
    assert type(qmodel[0]) is qtype
    state = qmodel.state_dict()
    codes = [k for k in state if k.endswith("_int8")]
    assert codes and all(state[k].dtype == np.int8 for k in codes)
    assert not [k for k in state if ".weight" in k and not k.endswith(("_int8", "_scale", "_zero_point"))]
    assert type(model[0]) is not qtype   # the float module is left alone
    x = _dev(gpu, np.random.default_rng(0).standard_normal(shape))

    def first(o):
        return o[0] if isinstance(o, tuple) else o

    want = first(model(x)).numpy().astype(np.float64)
    got = first(qmodel(x)).numpy().astype(np.float64)
    assert np.abs(got - want).mean() / (np.abs(want).mean() + 1e-9) < 0.03


def test_default_spec_quantizes_every_recurrent_type(gpu):
    # test_dynamic_recurrent.py:116-121
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.quantization import quantize_dynamic

    model = nn.Sequential(nn.GRU(4, 4), nn.LSTMCell(4, 4), nn.GRUCell(4, 4), nn.RNNCell(4, 4)).to("gpu")
    q = quantize_dynamic(model)
    assert [type(m) for m in q] == [nnqd.GRU, nnqd.LSTMCell, nnqd.GRUCell, nnqd.RNNCell]


def test_spec_filters_recurrent_types(gpu):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.quantization import quantize_dynamic

    model = nn.Sequential(nn.GRU(4, 4), nn.GRUCell(4, 4)).to("gpu")
    q = quantize_dynamic(model, qconfig_spec={nn.GRUCell})
    assert type(q[0]) is nn.GRU and type(q[1]) is nnqd.GRUCell


def test_from_float_rejects_another_type(gpu):
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd

    with pytest.raises(TypeError):
        nnqd.LSTM.from_float(nn.GRU(4, 4))


# ------------------------------------------------------------------ packed sequences


def test_pack_pad_round_trip(gpu):
    """pack_padded_sequence / pad_packed_sequence / pack_sequence / pad_sequence as row moves:
    bit-exact round trips, sorted and unsorted, time- and batch-major (lucid/nn/utils/rnn.py:
    394-777); batch_sizes, the permutations and the returned lengths as Lucid documents them."""
    from lucid_amd.nn.utils.rnn import pack_padded_sequence, pack_sequence, pad_packed_sequence, pad_sequence

    rng = np.random.default_rng(2)
    T, B, F = 6, 4, 5
    lens = [3, 6, 2, 5]
    x = rng.standard_normal((T, B, F)).astype(np.float32)
    for batch_first in (False, True):
        xin = x.transpose(1, 0, 2) if batch_first else x
        p = pack_padded_sequence(_dev(gpu, xin), lens, batch_first=batch_first, enforce_sorted=False)
        assert p.batch_sizes.numpy().tolist() == [4, 4, 3, 2, 2, 1]
        assert p.sorted_indices.numpy().tolist() == [1, 3, 0, 2]
        assert p.unsorted_indices.numpy().tolist() == [2, 0, 3, 1]
        rows = [x[t, b] for t in range(T) for b in [1, 3, 0, 2] if lens[b] > t]
        np.testing.assert_array_equal(p.data.numpy(), np.stack(rows))
        padded, got_lens = pad_packed_sequence(p, batch_first=batch_first, padding_value=-7.0)
        want = xin.copy()
        for b, n in enumerate(lens):
            if batch_first:
                want[b, n:] = -7.0
            else:
                want[n:, b] = -7.0
        np.testing.assert_array_equal(padded.numpy(), want)
        assert got_lens.numpy().tolist() == lens
    with pytest.raises(ValueError, match="sorted in decreasing order"):
        pack_padded_sequence(_dev(gpu, x), lens)
    seqs = [_dev(gpu, rng.standard_normal((n, F)).astype(np.float32)) for n in (5, 5, 2)]
    ps = pack_sequence(seqs)
    assert ps.batch_sizes.numpy().tolist() == [3, 3, 2, 2, 2]
    padded = pad_sequence(seqs, batch_first=True, padding_value=1.5).numpy()
    np.testing.assert_array_equal(padded[2, :2], seqs[2].numpy())
    assert np.all(padded[2, 2:] == 1.5)


@pytest.mark.parametrize("mode,layers,bidir", [("LSTM", 2, True), ("GRU", 1, False), ("LSTM", 1, False),
                                               ("GRU", 2, True)])
@pytest.mark.parametrize("dynamic", [False, True])
def test_packed_sequence_recurrence(gpu, mode, layers, bidir, dynamic):
    """An unsorted PackedSequence through LSTM / GRU (float and dynamic int8): each sequence's
    outputs and final states equal the oracle's float64 recurrence over that sequence alone
    (the packed recurrence advances only the live sequences at each step), within 2e-5; the
    output comes back packed with the input's batch sizes and permutations."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.nn.layers import manual_seed
    from lucid_amd.nn.utils.rnn import PackedSequence, pack_padded_sequence, pad_packed_sequence

    manual_seed(11 + layers)
    rng = np.random.default_rng(layers + 2 * bidir)
    T, B, I, H = 7, 5, 6, 8
    lens = [4, 7, 1, 7, 3]
    D = 2 if bidir else 1
    m = getattr(nn, mode)(I, H, num_layers=layers, bidirectional=bidir).to("gpu")
    mod = nnqd.__dict__[mode].from_float(m) if dynamic else m
    weights = _deq_weights(mod) if dynamic else _float_weights(m)
    x = rng.standard_normal((T, B, I)).astype(np.float32)
    h0 = (rng.standard_normal((layers * D, B, H)) * 0.5).astype(np.float32)
    c0 = (rng.standard_normal((layers * D, B, H)) * 0.5).astype(np.float32)
    packed = pack_padded_sequence(_dev(gpu, x), lens, enforce_sorted=False)
    hx = (_dev(gpu, h0), _dev(gpu, c0)) if mode == "LSTM" else _dev(gpu, h0)
    out, state = mod(packed, hx)
    assert isinstance(out, PackedSequence)
    assert out.batch_sizes.numpy().tolist() == packed.batch_sizes.numpy().tolist()
    padded, got_lens = pad_packed_sequence(out)
    assert got_lens.numpy().tolist() == lens
    h_n = state[0].numpy() if mode == "LSTM" else state.numpy()
    for b, n in enumerate(lens):
        want, wh, wc = O.rnn_forward(mode, x[:n, b:b + 1], weights, layers, bidir, h0[:, b:b + 1],
                                     c0[:, b:b + 1] if mode == "LSTM" else None)
        np.testing.assert_allclose(padded.numpy()[:n, b:b + 1], want, atol=ATOL, rtol=0)
        assert np.all(padded.numpy()[n:, b] == 0.0)
        np.testing.assert_allclose(h_n[:, b:b + 1], wh, atol=ATOL, rtol=0)
        if mode == "LSTM":
            np.testing.assert_allclose(state[1].numpy()[:, b:b + 1], wc, atol=ATOL, rtol=0)


@pytest.mark.parametrize("layers,bidir,batch_first,packed", [(1, False, True, False), (2, True, False, False),
                                                             (2, True, False, True), (1, False, False, True)])
@pytest.mark.parametrize("dynamic", [False, True])
def test_projected_lstm(gpu, layers, bidir, batch_first, packed, dynamic):
    """LSTM with proj_size P (lucid/nn/modules/recurrent_base.py:138-192; the engine's projected
    step, lucid/_C/backend/cpu/Lstm.h:90-164): weight_hr [P, H] after each layer's biases,
    weight_hh [4H, P], outputs and h_n P wide, c_n H wide.  Float and dynamic int8 (weight_hr
    quantized like every weight) against the oracle's float64 recurrence, 2e-5; dense and
    unsorted packed input; h_n is the last step of the output (the reference's own check,
    lucid/test/unit/nn/test_recurrent.py:54-66)."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd
    from lucid_amd.nn.layers import manual_seed
    from lucid_amd.nn.utils.rnn import pack_padded_sequence, pad_packed_sequence

    manual_seed(40 + layers)
    rng = np.random.default_rng(7 * layers + bidir)
    T, B, I, H, P = 6, 4, 5, 12, 3
    D = 2 if bidir else 1
    m = nn.LSTM(I, H, num_layers=layers, bidirectional=bidir, batch_first=batch_first, proj_size=P).to("gpu")
    names = [n for n, _ in m.named_parameters()]
    assert names[:5] == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "weight_hr_l0"]
    mod = nnqd.LSTM.from_float(m) if dynamic else m
    if dynamic:
        assert "weight_hr_l0_int8" in dict(mod.named_buffers())
    weights = _deq_weights(mod) if dynamic else _float_weights(m)
    x = rng.standard_normal((T, B, I)).astype(np.float32)
    h0 = (rng.standard_normal((layers * D, B, P)) * 0.5).astype(np.float32)
    c0 = (rng.standard_normal((layers * D, B, H)) * 0.5).astype(np.float32)
    hx = (_dev(gpu, h0), _dev(gpu, c0))
    if packed:
        lens = [3, 6, 1, 5]
        out, (h_n, c_n) = mod(pack_padded_sequence(_dev(gpu, x), lens, enforce_sorted=False), hx)
        padded, _ = pad_packed_sequence(out)
        got, h_n, c_n = padded.numpy(), h_n.numpy(), c_n.numpy()
        for b, n in enumerate(lens):
            want, wh, wc = O.rnn_forward("LSTM", x[:n, b:b + 1], weights, layers, bidir, h0[:, b:b + 1],
                                         c0[:, b:b + 1])
            np.testing.assert_allclose(got[:n, b:b + 1], want, atol=ATOL, rtol=0)
            np.testing.assert_allclose(h_n[:, b:b + 1], wh, atol=ATOL, rtol=0)
            np.testing.assert_allclose(c_n[:, b:b + 1], wc, atol=ATOL, rtol=0)
        return
    xin = x.transpose(1, 0, 2) if batch_first else x
    out, (h_n, c_n) = mod(_dev(gpu, xin), hx)
    assert tuple(out.shape) == ((B, T, D * P) if batch_first else (T, B, D * P))
    assert tuple(h_n.shape) == (layers * D, B, P) and tuple(c_n.shape) == (layers * D, B, H)
    got = out.numpy().transpose(1, 0, 2) if batch_first else out.numpy()
    want, wh, wc = O.rnn_forward("LSTM", x, weights, layers, bidir, h0, c0)
    np.testing.assert_allclose(got, want, atol=ATOL, rtol=0)
    np.testing.assert_allclose(h_n.numpy(), wh, atol=ATOL, rtol=0)
    np.testing.assert_allclose(c_n.numpy(), wc, atol=ATOL, rtol=0)
    np.testing.assert_array_equal(h_n.numpy()[(layers - 1) * D], got[-1, :, :P])
