"""Write the golden fixtures of the quantized path (run: python tests/golden/make_golden.py).

Lucid's own test suite holds no quantized golden vectors (its only .npz goldens are
fp32 matmul/linear/softmax, lucid/test/numerical/golden/), and its package cannot be
imported here (it needs Python >= 3.14 and macOS).  Its parity suite pins the quantized
primitives against PyTorch (lucid/test/parity/quantization/test_functional_parity.py,
test_observer_parity.py), so these fixtures are PyTorch's outputs on seeded inputs --
an independent implementation of the same arithmetic -- plus the reference's inline
known-answer vectors (lucid/test/unit/quantization/test_functional.py,
test_observer.py).  Each array is data: inputs and expected outputs.
"""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def torch_fixtures() -> dict[str, np.ndarray]:
    import torch

    out: dict[str, np.ndarray] = {}
    rng = np.random.default_rng(20261201)
    # per-tensor quantize: (scale, zero point, dtype) cases over one input with outliers
    x = rng.standard_normal(4096).astype(np.float32)
    x[rng.choice(4096, 16, replace=False)] *= 20.0
    out["pt_x"] = x
    cases = [(0.05, 0, "qint8"), (0.037, 3, "qint8"), (0.0123, -7, "qint8"),
             (0.02, 128, "quint8"), (0.07, 0, "quint8"), (0.3333, 200, "quint8")]
    out["pt_scale"] = np.array([c[0] for c in cases], np.float64)
    out["pt_zp"] = np.array([c[1] for c in cases], np.int64)
    out["pt_signed"] = np.array([c[2] == "qint8" for c in cases])
    codes, fq = [], []
    for s, z, dt in cases:
        tdt = torch.qint8 if dt == "qint8" else torch.quint8
        q = torch.quantize_per_tensor(torch.from_numpy(x), s, z, tdt)
        codes.append(q.int_repr().numpy().astype(np.int16))
        qmin, qmax = (-128, 127) if dt == "qint8" else (0, 255)
        fq.append(torch.fake_quantize_per_tensor_affine(torch.from_numpy(x), s, z, qmin, qmax)
                  .numpy())
    out["pt_codes"] = np.stack(codes)
    out["pt_fake"] = np.stack(fq)
    out["pt_dequant"] = np.stack([
        torch.quantize_per_tensor(torch.from_numpy(x), s, z,
                                  torch.qint8 if dt == "qint8" else torch.quint8)
        .dequantize().numpy() for s, z, dt in cases])

    # per-channel quantize along axis 0 and 1 of a [48, 64] weight
    w = rng.standard_normal((48, 64)).astype(np.float32)
    out["pc_w"] = w
    for axis in (0, 1):
        C = w.shape[axis]
        sc = rng.uniform(0.005, 0.05, C).astype(np.float32)
        zp = np.zeros(C, np.int64)
        q = torch.quantize_per_channel(torch.from_numpy(w), torch.from_numpy(sc.astype(np.float64)),
                                       torch.from_numpy(zp), axis, torch.qint8)
        out[f"pc{axis}_scale"] = sc
        out[f"pc{axis}_codes"] = q.int_repr().numpy()
        out[f"pc{axis}_fake"] = torch.fake_quantize_per_channel_affine(
            torch.from_numpy(w), torch.from_numpy(sc), torch.from_numpy(zp.astype(np.int32)), axis,
            -128, 127).numpy()

    # observers: three batches, reference observers' qparams
    from torch.ao.quantization import observer as tobs

    batches = [rng.standard_normal((4, 8)).astype(np.float32) for _ in range(3)]
    out["obs_batches"] = np.stack(batches)
    mm = tobs.MinMaxObserver(dtype=torch.quint8, qscheme=torch.per_tensor_affine)
    ema = tobs.MovingAverageMinMaxObserver(averaging_constant=0.1, dtype=torch.quint8,
                                           qscheme=torch.per_tensor_affine)
    for b in batches:
        mm(torch.from_numpy(b))
        ema(torch.from_numpy(b))
    s, z = mm.calculate_qparams()
    out["obs_minmax_scale"], out["obs_minmax_zp"] = s.numpy(), z.numpy()
    out["obs_minmax_range"] = np.array([mm.min_val.item(), mm.max_val.item()], np.float32)
    s, z = ema.calculate_qparams()
    out["obs_ema_scale"], out["obs_ema_zp"] = s.numpy(), z.numpy()
    pc = tobs.PerChannelMinMaxObserver(ch_axis=0, dtype=torch.qint8,
                                       qscheme=torch.per_channel_symmetric)
    pw = rng.standard_normal((6, 10)).astype(np.float32)
    pc(torch.from_numpy(pw))
    s, _ = pc.calculate_qparams()
    out["obs_pc_x"], out["obs_pc_scale"] = pw, s.numpy()
    return out


def main() -> None:
    fx = torch_fixtures()
    path = os.path.join(HERE, "torch_quant.npz")
    np.savez_compressed(path, **fx)
    print(f"wrote {path}: {sorted(fx)}")


if __name__ == "__main__":
    main()
