"""Counterpart of Lucid's ``tools/bench_quantized_dispatch.py`` on the HIP backend.

``python -m lucid_amd.bench_quantized_dispatch --output report.json [--iter 20] [--width 1024]``

Same protocol as the reference harness (tools/bench_quantized_dispatch.py:26-105 with
tools/_bench_timing.py:33-52): for bits in (4, 8), a ``width x width`` float weight is
group-wise quantized (group 64); for batch M in (1, 2, 8, 32) and x of shape (M, width):

* the parity gate ``max|cached - packed| / max|cached| <= 1e-4`` runs before any timing;
* three paths are timed: ``packed`` (``quantized_matmul`` on the packed weight),
  ``cached_dense`` (``x @ dense^T`` with the dequantized weight kept) and
  ``dequant_each_call`` (dequantize, then the dense product, every call);
* each path: one cold call, 5 warm-ups, ``--iter`` timed calls, each call materialized
  (device synchronize) -- median / p5 / p95 in ms.

Rows carry the reference's keys plus the throughput view: GB/s of the weight bytes the
path reads, its fraction of the 8 TB/s HBM3E peak, TOPS, and the host core count.  The
random streams differ from Lucid's (``lucid.manual_seed`` + ``lucid.randn`` are engine
internals); inputs are standard normal from numpy's generator with the same seed.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import time
from pathlib import Path

import numpy as np

HBM_PEAK_GBS = 8000.0


def _materialize(C) -> None:
    C.synchronize()


def cold_ms(C, call) -> float:
    C.synchronize()
    t0 = time.perf_counter()
    call()
    _materialize(C)
    return (time.perf_counter() - t0) * 1000.0


def warm_ms(C, call, n_warmup: int, n_iter: int) -> tuple[float, float, float]:
    if n_warmup < 0 or n_iter < 1:
        raise ValueError("warmup must be nonnegative and iterations must be positive")
    for _ in range(n_warmup):
        call()
    C.synchronize()
    samples = sorted(cold_ms(C, call) for _ in range(n_iter))
    return (statistics.median(samples), samples[min(n_iter - 1, int(n_iter * 0.05))],
            samples[min(n_iter - 1, int(n_iter * 0.95))])


def run(iters: int = 20, width: int = 1024, seed: int = 20260920, verbose: bool = True) -> dict:
    import lucid_amd as L
    from lucid_amd import _C as C
    from lucid_amd.nn import functional as F
    from lucid_amd.quantization import _qgemm

    if not L.is_available():
        raise RuntimeError("no HIP device visible")
    rng = np.random.default_rng(seed)
    rows = []
    for bits in (4, 8):
        weight = L.tensor(rng.standard_normal((width, width)).astype(np.float32), device="gpu")
        packed, scales, biases = _qgemm.quantize(weight, group_size=64, bits=bits)
        dense = _qgemm.dequantize(packed, scales, biases, group_size=64, bits=bits)
        for batch in (1, 2, 8, 32):
            x = L.tensor(rng.standard_normal((batch, width)).astype(np.float32), device="gpu")

            def packed_call():
                return _qgemm.quantized_matmul(x, packed, scales, biases, transpose=True,
                                               group_size=64, bits=bits)

            def cached_call():
                return F.linear(x, dense)

            def unpack_call():
                w = _qgemm.dequantize(packed, scales, biases, group_size=64, bits=bits)
                return F.linear(x, w)

            expected, actual = cached_call().numpy(), packed_call().numpy()
            error = float(np.max(np.abs(expected.astype(np.float64) - actual)))
            scale = max(float(np.max(np.abs(expected))), 1e-12)
            if not error / scale <= 1e-4:
                raise RuntimeError(f"parity failure for bits={bits}, M={batch}: {error / scale}")
            wbytes = {"packed": width * width * bits / 8 + 8.0 * width * (width // 64),
                      "cached_dense": 4.0 * width * width,
                      "dequant_each_call": width * width * bits / 8 + 8.0 * width * (width // 64)
                      + 8.0 * width * width}
            for name, call in (("packed", packed_call), ("cached_dense", cached_call),
                               ("dequant_each_call", unpack_call)):
                first = cold_ms(C, call)
                median, p5, p95 = warm_ms(C, call, 5, iters)
                moved = wbytes[name] + 4.0 * batch * 2 * width
                gbs = moved / (median * 1e-3) / 1e9
                row = {
                    "bits": bits, "m": batch, "n": width, "k": width, "path": name,
                    "first_ms": first, "median_ms": median, "p5_ms": p5, "p95_ms": p95,
                    "parity_relative_error": error / scale,
                    "TOPS": 2.0 * batch * width * width / (median * 1e-3) / 1e12,
                    "GB/s": gbs, "hbm_roofline_frac": gbs / HBM_PEAK_GBS,
                    "host_cores": os.cpu_count(),
                }
                rows.append(row)
                if verbose:
                    print(json.dumps(row), flush=True)
    return {
        "environment": {"platform": platform.platform(), "python": platform.python_version(),
                        "device": "AMD Instinct MI355X (gfx950)",
                        "backend": C.lib().lq_backend_name().decode(),
                        "host_cores": os.cpu_count()},
        "contract": "end-to-end per-call materialization and sync; 5 warmups; first call is "
                    "not cold compilation",
        "iterations": iters,
        "rows": rows,
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--output", type=Path, required=True)
    parser.add_argument("--iter", type=int, default=20)
    parser.add_argument("--width", type=int, default=1024)
    args = parser.parse_args()
    if args.iter < 1 or args.width < 64 or args.width % 64:
        parser.error("iterations must be positive and width a positive multiple of 64")
    report = run(args.iter, args.width)
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(report, indent=2, allow_nan=False) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
