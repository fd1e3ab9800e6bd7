"""Decode-GEMV route comparison: ``python -m lucid_amd.bench_gemv [--iters N]``.

For the weight-only int8 GEMV at the decode shapes (M = 1, 16 over 4096 x 4096, 11008 x 4096,
4096 x 11008; weights rotated past the 256 MB Infinity Cache) it times, by HIP-graph replay:

* ``lq_gemv_w8`` without a workspace (for 3 <= M: the one-kernel route, each workgroup 16 weight
  rows and all of K, splitting x itself);
* ``lq_gemv_w8`` with its workspace (from 12 rows: the split-K route, x split once per 64
  columns and K range);
* ``lq_gemv_w8_packed`` (the MFMA-packed weight nnq.Linear uses for 3..16 rows);
* a streaming-read floor: the min/max observer (``lq_minmax_f32``) over as many bytes as the
  weight, i.e. one launch that only reads them.

One JSON line per shape.  ``rocprofv3 --kernel-trace --stats`` / ``--pmc`` around this module
give the per-kernel times and counters of each route (kernel names differ per route).
"""

from __future__ import annotations

import argparse
import ctypes
import json

import numpy as np


def _rotations(nbytes: int) -> int:
    return max(1, -(-(512 << 20) // max(nbytes, 1)))


def main() -> None:
    import lucid_amd as L
    from lucid_amd import _C as C

    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--shapes", default="1x4096x4096,16x4096x4096,1x11008x4096,16x11008x4096,16x4096x11008")
    args = ap.parse_args()
    lib = C.lib()
    stream = ctypes.c_void_p()
    C.call("lq_stream_create", ctypes.byref(stream))
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    C.call("lq_event_create", ctypes.byref(ev0))
    C.call("lq_event_create", ctypes.byref(ev1))

    def graph_us(calls, reps):
        C.call("lq_graph_begin_capture", stream)
        for c in calls:
            c(stream)
        exe = ctypes.c_void_p()
        C.call("lq_graph_end_capture", stream, ctypes.byref(exe))
        for _ in range(2):
            C.call("lq_graph_launch", exe, stream)
        C.call("lq_stream_synchronize", stream)
        C.call("lq_event_record", ev0, stream)
        for _ in range(reps):
            C.call("lq_graph_launch", exe, stream)
        C.call("lq_event_record", ev1, stream)
        C.call("lq_event_synchronize", ev1)
        ms = ctypes.c_float()
        C.call("lq_event_elapsed_ms", ctypes.byref(ms), ev0, ev1)
        C.call("lq_graph_destroy", exe)
        return ms.value * 1e3 / (reps * len(calls))

    rng = np.random.default_rng(3)
    for spec in args.shapes.split(","):
        M, N, K = (int(v) for v in spec.split("x"))
        rot = _rotations(N * K)
        W = L.empty((rot * N * K,), np.int8, "gpu")
        C.call("lq_fill_u32", W.data_ptr(), 0x3A1F05C7, rot * N * K // 4, None)
        pb = lib.lq_packed_weights_size(N, K)
        P = L.empty((rot * pb,), np.int8, "gpu")
        for r in range(rot):
            C.call("lq_pack_weights_i8", W.data_ptr() + r * N * K, K, N, K, P.data_ptr() + r * pb, None)
        x = L.tensor(rng.standard_normal((M, K)).astype(np.float32), device="gpu")
        y = L.empty((M, N), np.float32, "gpu")
        s = L.tensor(rng.uniform(1e-3, 1e-1, N).astype(np.float32), device="gpu")
        wsb = lib.lq_gemv_w8_workspace_size(M, N, K)
        ws = L.empty((max(wsb, 1),), np.uint8, "gpu")
        pws = lib.lq_gemv_w8_packed_workspace_size(M, N, K)
        pw = L.empty((max(pws, 1),), np.uint8, "gpu")
        nbytes = N * K + 4.0 * N + 4.0 * M * (K + N)
        res = {"M": M, "N": N, "K": K, "weight_copies": rot}
        routes = {
            "no_workspace": lambda r, st: lib.lq_gemv_w8(x.data_ptr(), C.F32, K, W.data_ptr() + r * N * K, K,
                                                           s.data_ptr(), None, None, y.data_ptr(), N, M, N, K, 0,
                                                           None, 0, st),
            "workspace": lambda r, st: lib.lq_gemv_w8(x.data_ptr(), C.F32, K, W.data_ptr() + r * N * K, K,
                                                        s.data_ptr(), None, None, y.data_ptr(), N, M, N, K, 0,
                                                        ws.data_ptr(), wsb, st),
            "packed": lambda r, st: lib.lq_gemv_w8_packed(x.data_ptr(), C.F32, K, P.data_ptr() + r * pb,
                                                          s.data_ptr(), None, None, y.data_ptr(), N, M, N, K, 0,
                                                          pw.data_ptr(), pws, st),
        }
        for name, fn in routes.items():
            calls = [lambda st, r=r, fn=fn: C.check(fn(r, st), name) for r in range(rot)]
            us = graph_us(calls, args.iters)
            res[name] = {"us": round(us, 2), "frac_hbm": round(nbytes / (us * 1e-6) / 8e12, 3), "path": C.last_path()}
        # streaming-read floor: one observer launch over the same number of bytes (rotated)
        n = N * K // 4
        mn = L.tensor(np.float32(np.inf), device="gpu")
        mx = L.tensor(np.float32(-np.inf), device="gpu")
        owb = lib.lq_minmax_workspace_size(n)
        ow = L.empty((max(owb, 1),), np.uint8, "gpu")
        calls = [lambda st, r=r: C.call("lq_minmax_f32", W.data_ptr() + r * N * K, n, mn.data_ptr(), mx.data_ptr(),
                                        C.OBS_REPLACE, 0.0, ow.data_ptr(), owb, st) for r in range(rot)]
        us = graph_us(calls, args.iters)
        res["stream_floor"] = {"us": round(us, 2), "frac_hbm": round(N * K / (us * 1e-6) / 8e12, 3),
                               "kernel": "lq_minmax_f32 over the weight's bytes"}
        print(json.dumps(res), flush=True)
        del W, P


if __name__ == "__main__":
    main()
