"""CPU oracle for the int8 quantized-inference path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker / the timed CPU baseline.  The
product package ``lucid_amd`` never imports it.

Thin numpy wrappers over ``liblq_oracle.so`` (built from ``lq_oracle.c`` by
``oracle/Makefile``), a plain-C restatement of Lucid's arithmetic:

============================  ==========================================================
function                      follows (lucid-official/lucid)
============================  ==========================================================
``rne``                       ``lucid.round`` = vvnintf (backend/cpu/methods/Unary.cpp:143-147)
``clip``                      backend/cpu/Vdsp.cpp:33-62 (NaN passes, signed-zero ties)
``minmax`` / ``_per_channel``  observer.py:408-414, 527-544, 672-685, 1031-1048;
                              backend/cpu/Reduce.cpp:54-105
``calc_qparams``              quantization/_qparams.py:186-205
``quantize``                  quantization/_functional.py:59-69, 179-197
``dequantize``                quantization/_functional.py:281-293
``fake_quantize``             quantization/_functional.py:314-333
``gemm_w8a8``                 build-defined integer contract (no reference counterpart):
                              exact int32 sum, then the epilogue documented in
                              include/lq_api.h; int32 core checked by brute force
``conv2d_acc``                exact int64 brute force of the int8 conv sum (no reference
                              counterpart); padding modes as nn/functional/conv.py:24-29,76-81
``conv2d_f32``                float conv, per output sum over (c, kh, kw) in float32
                              (backend/cpu/methods/Conv.cpp:271-360 computes it by im2col +
                              sgemm: tolerance parity; bit-exact against the GPU's op order)
``linear``                    F.linear (nn/functional/linear.py:23-93 -> backend/cpu/methods/
                              Matmul.cpp:80-122: sgemm with W transposed, then the bias
                              add) in float64 (tolerance reference: sgemm's summation order
                              is not knowable); pinned by the reference's own goldens
                              lucid/test/numerical/golden/{linear_2x4_4to3,matmul_4x4}.npz
``gemv_w8``                   nn/quantized/linear.py:206-210 (dequantize -> F.linear) with
                              float64 accumulation (tolerance reference)
``group_*``                   quantization/_qgemm.py:84-97, 167-170 (MLX 0.32.3 internals:
                              parity unpinned beyond this documented formula);
                              ``group_matmul`` adds the dtype rule of QuantizedMatmul.cpp:153-164
                              and mlx_linear.py:215-222 (``round_to`` / ``bf16_round``)
``histc``                     _ops/_adapters.py:1256-1279 -> backend/cpu/methods/
                              Reduction.cpp:839-884 (double-precision bins, numpy)
``hist_rebin``                quantization/observer.py:826-848 (float32 centers / index,
                              sequential scatter_add, numpy)
``histogram_observer``        observer.py:850-870 (forward over batches)
``hist_clip_search``          observer.py:872-926, vectorised (cumulative sums and array
                              errors instead of the reference's Python loops)
``activation``                backend/cpu/methods/Activation.cpp:8-50, 375-460, 661-751;
                              Unary.cpp:165-170 (numpy float32; exp / tanh within rounding)
``embedding_bag``             backend/cpu/methods/Sequence.cpp:8-93 (bags: IndexBounds.h:107-150;
                              per_sample_weights: nn/functional/sparse.py:228-310)
``pool2d``                    backend/cpu/Pool.cpp:27-168; adaptive cells nn/functional/
                              _pool_core.py:228-250 (numpy)
``rnn_cell`` / ``rnn_forward``  nn/modules/rnn.py (_rnn_step, _gru_step, LSTM gates i, f, g, o),
                              float64 numpy
``conv_transpose2d_acc``      the direct scatter definition of conv_transpose2d, int64
``layer_norm`` / ``gelu_tanh`` /  the float glue of the int8 decoder:
``attention`` / ``embedding_sum``  nn.LayerNorm, F.gelu(approximate="tanh"),
                              F.scaled_dot_product_attention(is_causal) over fp16 q / k / v,
                              token + position embedding; float64 numpy (tolerance references)
``lucid_*``                   the multi-pass CPU composition timed as the CPU baseline
============================  ==========================================================

Pins (tests/test_oracle.py): the reference's known-answer tests, torch's
``quantize_per_tensor`` / ``fake_quantize_per_*`` (the independent oracle the
reference's own parity suite uses), closed forms and brute force.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblq_oracle.so")

# Element-type codes shared with include/lq_api.h.
I8, U8, I16, I32, F16, F32, U8S8 = 1, 2, 3, 4, 5, 6, 7
OBS_MINMAX, OBS_EMA, OBS_REPLACE = 0, 1, 2
OUT_I32, OUT_F32, OUT_F16, OUT_Q8, OUT_QU8, OUT_FQ32, OUT_Q16, OUT_QU8S8 = 0, 1, 2, 3, 4, 5, 6, 7

_CODE_NP = {I8: np.int8, U8: np.uint8, I16: np.int16, I32: np.int32, U8S8: np.int8}

_lib = None


def build() -> None:
    """Compile ``liblq_oracle.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    L.lqo_rne.argtypes, L.lqo_rne.restype = [_F], _F
    L.lqo_clip.argtypes, L.lqo_clip.restype = [_F, _F, _F], _F
    L.lqo_extreme.argtypes, L.lqo_extreme.restype = [_F, _F, _I], _F
    L.lqo_f32_to_f16.argtypes, L.lqo_f32_to_f16.restype = [_F], ctypes.c_uint16
    L.lqo_recip_f32.argtypes, L.lqo_recip_f32.restype = [_F], _F
    L.lqo_recip_f64.argtypes, L.lqo_recip_f64.restype = [ctypes.c_double], _F
    L.lqo_minmax.argtypes = [_P, _I64, _P, _I, _F]
    L.lqo_minmax_per_channel.argtypes = [_P, _I64, _I64, _I64, _P, _P, _I, _F]
    L.lqo_calc_qparams.argtypes = [_P, _P, _I64, _I, _I, _I, _I, _F, _P, _P]
    L.lqo_quantize.argtypes = [_P, _I64, _I64, _I64, _P, _P, _I, _I, _P, _I]
    L.lqo_dequantize.argtypes = [_P, _I, _I64, _I64, _I64, _P, _P, _P, _I]
    L.lqo_fake_quantize.argtypes = [_P, _I64, _I64, _I64, _P, _P, _P, _I, _I, _P, _P]
    L.lqo_gemm_acc.argtypes = [_P, _I64, _P, _I64, _I64, _I64, _I64, ctypes.c_int32, _P, _P]
    L.lqo_gemm_acc.restype = _I
    L.lqo_gemm_w8a8.argtypes = [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P,
                                _I64, _F, _P, _P, _F, _F, _I, _I, _I, _I]
    L.lqo_gemm_w8a8.restype = _I
    L.lqo_gemm_epilogue.argtypes = [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _F, _F, _I, _I, _I, _I,
                                    _P, _I64]
    L.lqo_gemv_w8.argtypes = [_P, _I64, _I64, _P, _I64, _P, _P, _P, _I, _P]
    L.lqo_conv2d_acc.argtypes = [_P, _I, _I, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I, _I,
                                 _I, _I, _I, _I, _I, _I, _I64, _I, _P]
    L.lqo_conv2d_acc.restype = _I
    L.lqo_conv2d_f32.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I, _I, _I,
                                 _I, _I, _I, _I, _I, _I64, _I, _P]
    L.lqo_group_quantize.argtypes = [_P, _I64, _I64, _I, _I, _P, _P, _P]
    L.lqo_group_dequantize.argtypes = [_P, _P, _P, _I64, _I64, _I, _I, _P]
    L.lqo_lucid_minmax.argtypes = [_P, _I64, _P, _P]
    L.lqo_lucid_quantize.argtypes = [_P, _I64, _F, _F, _I, _I, _P, _P, _P]
    L.lqo_lucid_dequantize.argtypes = [_P, _I64, _F, _F, _P, _P]
    L.lqo_set_threads.argtypes, L.lqo_set_threads.restype = [_I], _I
    L.lqo_div6_mismatches.argtypes, L.lqo_div6_mismatches.restype = [], _I64


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32, order="C")


# ---------------------------------------------------------------- scalar rules


def rne(x: float) -> float:
    return lib().lqo_rne(x)


def clip(v: float, lo: float, hi: float) -> float:
    return lib().lqo_clip(v, lo, hi)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = _f32(x).ravel()
    return np.array([L.lqo_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def recip_tensor(s) -> np.ndarray:
    """Reciprocal of a float32 tensor scale: 1.0f / s in float32."""
    s = _f32(s)
    return (np.float32(1.0) / s).astype(np.float32)


def recip_scalar(s: float) -> np.float32:
    """Reciprocal of a Python-float scale: fl32(1.0 / s) computed in double."""
    return np.float32(lib().lqo_recip_f64(float(s)))


# ------------------------------------------------------------------ observers


def minmax(x: np.ndarray, running=(np.inf, -np.inf), mode: int = OBS_MINMAX, c: float = 0.0):
    x = _f32(x).ravel()
    r = _f32(running).copy()
    lib().lqo_minmax(_ptr(x), x.size, _ptr(r), mode, np.float32(c))
    return r


def _ocl(shape, ch_axis):
    shape = tuple(shape)
    outer = int(np.prod(shape[:ch_axis], dtype=np.int64))
    C = int(shape[ch_axis])
    inner = int(np.prod(shape[ch_axis + 1 :], dtype=np.int64))
    return outer, C, inner


def minmax_per_channel(x: np.ndarray, ch_axis: int, rmin=None, rmax=None,
                       mode: int = OBS_MINMAX, c: float = 0.0):
    x = _f32(x)
    outer, C, inner = _ocl(x.shape, ch_axis)
    rmin = np.full(C, np.inf, np.float32) if rmin is None else _f32(np.broadcast_to(rmin, (C,))).copy()
    rmax = np.full(C, -np.inf, np.float32) if rmax is None else _f32(np.broadcast_to(rmax, (C,))).copy()
    lib().lqo_minmax_per_channel(_ptr(x), outer, C, inner, _ptr(rmin), _ptr(rmax), mode,
                                 np.float32(c))
    return rmin, rmax


def calc_qparams(mn, mx, symmetric: bool, signed: bool, qmin: int, qmax: int, eps: float = 1e-8):
    mn = _f32(mn)
    mx = _f32(mx)
    shape = mn.shape
    mn, mx = mn.ravel().copy(), mx.ravel().copy()
    s = np.empty_like(mn)
    z = np.empty_like(mn)
    lib().lqo_calc_qparams(_ptr(mn), _ptr(mx), mn.size, int(symmetric), int(signed), qmin, qmax,
                           np.float32(eps), _ptr(s), _ptr(z))
    return s.reshape(shape), z.reshape(shape)


# ----------------------------------------------------- quantize / dequantize


def _qp_vectors(C, inv, zp):
    inv = _f32(np.broadcast_to(np.asarray(inv, np.float32), (C,))).copy()
    zp = _f32(np.broadcast_to(np.asarray(zp, np.float32), (C,))).copy()
    return inv, zp


def quantize(x: np.ndarray, inv, zp, qmin: int, qmax: int, q_dtype: int = I8,
             ch_axis: int | None = None) -> np.ndarray:
    """Codes of ``x``; ``inv`` is the reciprocal already rounded to float32."""
    x = _f32(x)
    if ch_axis is None:
        outer, C, inner = 1, 1, x.size
    else:
        outer, C, inner = _ocl(x.shape, ch_axis)
    inv, zp = _qp_vectors(C, inv, zp)
    q = np.empty(x.shape, dtype=_CODE_NP[q_dtype])
    lib().lqo_quantize(_ptr(x), outer, C, inner, _ptr(inv), _ptr(zp), qmin, qmax, _ptr(q), q_dtype)
    return q


def dequantize(q: np.ndarray, q_dtype: int, s, zp, ch_axis: int | None = None,
               y_dtype: int = F32) -> np.ndarray:
    q = np.ascontiguousarray(q)
    if ch_axis is None:
        outer, C, inner = 1, 1, q.size
    else:
        outer, C, inner = _ocl(q.shape, ch_axis)
    s, zp = _qp_vectors(C, s, zp)
    if y_dtype == F16:
        y = np.empty(q.shape, np.uint16)
    else:
        y = np.empty(q.shape, np.float32)
    lib().lqo_dequantize(_ptr(q), q_dtype, outer, C, inner, _ptr(s), _ptr(zp), _ptr(y), y_dtype)
    return y.view(np.float16) if y_dtype == F16 else y


def fake_quantize(x: np.ndarray, inv, s, zp, qmin: int, qmax: int, ch_axis: int | None = None):
    x = _f32(x)
    if ch_axis is None:
        outer, C, inner = 1, 1, x.size
    else:
        outer, C, inner = _ocl(x.shape, ch_axis)
    inv, zp2 = _qp_vectors(C, inv, zp)
    s, _ = _qp_vectors(C, s, zp)
    y = np.empty_like(x)
    mask = np.empty_like(x)
    lib().lqo_fake_quantize(_ptr(x), outer, C, inner, _ptr(inv), _ptr(s), _ptr(zp2), qmin, qmax,
                            _ptr(y), _ptr(mask))
    return y, mask


# --------------------------------------------------------------------- GEMM


def gemm_acc(A: np.ndarray, B: np.ndarray, za: int = 0, zb=None) -> np.ndarray:
    """Exact int32 accumulator of sum_k (A[m,k]-za)(B[n,k]-zb[n]); B is [N,K]."""
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    N = B.shape[0]
    zbv = None if zb is None else np.ascontiguousarray(np.broadcast_to(zb, (N,)), np.int32)
    acc = np.empty((M, N), np.int32)
    ovf = lib().lqo_gemm_acc(_ptr(A), K, _ptr(B), K, M, N, K, int(za), _ptr(zbv), _ptr(acc))
    if ovf:
        raise OverflowError("int32 accumulator overflow")
    return acc


_OUT_NP = {OUT_I32: np.int32, OUT_F32: np.float32, OUT_F16: np.uint16, OUT_Q8: np.int8,
           OUT_QU8: np.uint8, OUT_FQ32: np.float32, OUT_Q16: np.int16, OUT_QU8S8: np.int8}


def gemm_w8a8(A, B, a_scale, b_scale, za=0.0, zb=None, bias=None, out_scale=1.0, out_zp=0.0,
              qmin=-128, qmax=127, out_kind=OUT_F32, relu=False) -> np.ndarray:
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    N = B.shape[0]
    a_scale = _f32(np.atleast_1d(a_scale))
    b_scale = _f32(np.atleast_1d(b_scale))
    a_stride = 0 if a_scale.size == 1 else 1
    b_stride = 0 if b_scale.size == 1 else 1
    zbv = None if zb is None else _f32(np.broadcast_to(zb, (N,)))
    bias = None if bias is None else _f32(bias)
    C = np.empty((M, N), _OUT_NP[out_kind])
    ovf = lib().lqo_gemm_w8a8(_ptr(A), K, _ptr(B), K, _ptr(C), N, M, N, K, _ptr(a_scale),
                              a_stride, _ptr(b_scale), b_stride, np.float32(za), _ptr(zbv),
                              _ptr(bias), np.float32(out_scale), np.float32(out_zp), qmin, qmax,
                              out_kind, int(relu))
    if ovf:
        raise OverflowError("int32 accumulator overflow")
    return C.view(np.float16) if out_kind == OUT_F16 else C


def gemm_epilogue(acc, a_scale, b_scale, bias=None, out_scale=1.0, out_zp=0.0, qmin=-128,
                  qmax=127, out_kind=OUT_F32, relu=False) -> np.ndarray:
    """The W8A8 epilogue applied to a precomputed int32 accumulator [M, N]."""
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    a_scale = _f32(np.atleast_1d(a_scale))
    b_scale = _f32(np.atleast_1d(b_scale))
    C = np.empty((M, N), _OUT_NP[out_kind])
    lib().lqo_gemm_epilogue(_ptr(acc), M, N, _ptr(a_scale), 0 if a_scale.size == 1 else 1,
                            _ptr(b_scale), 0 if b_scale.size == 1 else 1,
                            _ptr(None if bias is None else _f32(bias)), np.float32(out_scale),
                            np.float32(out_zp), qmin, qmax, out_kind, int(relu), _ptr(C), N)
    return C.view(np.float16) if out_kind == OUT_F16 else C


def linear(x, W, bias=None) -> np.ndarray:
    """y = x W^T + bias in float64 over float32 operands (F.linear's y = sgemm(x, W^T) then
    the bias add, Matmul.cpp:110-120).  Each product of two float32 values is exact in
    float64; the float64 sum carries far less error than a float32 sgemm, so the result is
    a tolerance reference for any float32 order."""
    xd = _f32(x).astype(np.float64)
    wd = _f32(W).astype(np.float64)
    y = xd @ wd.T
    if bias is not None:
        y = y + _f32(bias).astype(np.float64)
    return y


def gemv_w8(x, W, w_scale, w_zp=None, bias=None, relu=False) -> np.ndarray:
    x = _f32(x)
    W = np.ascontiguousarray(W, np.int8)
    M, K = x.shape
    N = W.shape[0]
    zb = None if w_zp is None else _f32(np.broadcast_to(w_zp, (N,)))
    y = np.empty((M, N), np.float64)
    lib().lqo_gemv_w8(_ptr(x), M, K, _ptr(W), N, _ptr(_f32(w_scale)), _ptr(zb),
                      _ptr(None if bias is None else _f32(bias)), int(relu), _ptr(y))
    return y


def conv_out_hw(H, W, KH, KW, stride, pad, dilation):
    sh, sw = stride
    pt, pb, pl, pr = pad
    dh, dw = dilation
    return ((H + pt + pb - dh * (KH - 1) - 1) // sh + 1, (W + pl + pr - dw * (KW - 1) - 1) // sw + 1)


def conv2d_acc(x, w, za=0, x_u8s8=False, stride=(1, 1), pad=(0, 0, 0, 0), dilation=(1, 1),
               groups=1, mode=0) -> np.ndarray:
    """Exact int32 conv accumulators [N, Cout, OH, OW] of codes x [N, C, H, W] (stored int8)
    and weight codes w [Cout, C/groups, KH, KW]; pad = (top, bottom, left, right)."""
    x = np.ascontiguousarray(x, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    N, C, H, W = x.shape
    Cout, _, KH, KW = w.shape
    OH, OW = conv_out_hw(H, W, KH, KW, stride, pad, dilation)
    acc = np.empty((N, Cout, OH, OW), np.int32)
    ovf = lib().lqo_conv2d_acc(_ptr(x), int(x_u8s8), int(za), N, C, H, W, _ptr(w), Cout, KH, KW,
                               stride[0], stride[1], pad[0], pad[1], pad[2], pad[3], dilation[0],
                               dilation[1], groups, mode, _ptr(acc))
    if ovf:
        raise OverflowError("int32 accumulator overflow")
    return acc


def conv2d_f32(x, w, bias=None, stride=(1, 1), pad=(0, 0, 0, 0), dilation=(1, 1), groups=1,
               mode=0) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    N, C, H, W = x.shape
    Cout, _, KH, KW = w.shape
    OH, OW = conv_out_hw(H, W, KH, KW, stride, pad, dilation)
    y = np.empty((N, Cout, OH, OW), np.float32)
    lib().lqo_conv2d_f32(_ptr(x), N, C, H, W, _ptr(w), _ptr(None if bias is None else _f32(bias)),
                         Cout, KH, KW, stride[0], stride[1], pad[0], pad[1], pad[2], pad[3],
                         dilation[0], dilation[1], groups, mode, _ptr(y))
    return y


def group_quantize(w, group_size: int, bits: int):
    w = _f32(w)
    N, K = w.shape
    packed = np.empty((N, K * bits // 32), np.uint32)
    scales = np.empty((N, K // group_size), np.float32)
    biases = np.empty((N, K // group_size), np.float32)
    lib().lqo_group_quantize(_ptr(w), N, K, group_size, bits, _ptr(packed), _ptr(scales),
                             _ptr(biases))
    return packed, scales, biases


def group_dequantize(packed, scales, biases, group_size: int, bits: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint32)
    N = packed.shape[0]
    K = packed.shape[1] * 32 // bits
    w = np.empty((N, K), np.float32)
    lib().lqo_group_dequantize(_ptr(packed), _ptr(_f32(scales)),
                               _ptr(None if biases is None else _f32(biases)), N, K, group_size,
                               bits, _ptr(w))
    return w


def group_codes(packed, bits: int) -> np.ndarray:
    """The codes c [N, K] of a packed weight: 32/bits codes per uint32, little end first."""
    packed = np.ascontiguousarray(packed, np.uint32)
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    c = (packed[:, :, None] >> shifts[None, None, :]) & np.uint32((1 << bits) - 1)
    return c.reshape(packed.shape[0], -1).astype(np.float64)


def bf16_round(x) -> np.ndarray:
    """Values rounded to bfloat16 precision (8 significant bits, float32's exponent range,
    round half to even, overflow to infinity), returned as float32.  One rounding from the
    given value (float32 or float64), written with frexp / rint in float64 (an arithmetic
    route, independent of bit tricks)."""
    x = np.asarray(x, np.float64)
    out = x.copy()
    fin = np.isfinite(x) & (x != 0)
    m, e = np.frexp(x[fin])                      # x = m 2^e, 0.5 <= |m| < 1
    ulp_e = np.maximum(e - 8, -133)              # spacing 2^(e-8); subnormal floor 2^-133
    out[fin] = np.rint(np.ldexp(x[fin], -ulp_e)) * np.ldexp(1.0, ulp_e)
    with np.errstate(over="ignore"):
        return out.astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """One rounding of the given values to 'f32', 'f16' or 'bf16' (Lucid's astype), kept as
    float64."""
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore"):
        if dtype == "f16":
            return x.astype(np.float16).astype(np.float64)
        if dtype == "bf16":
            return bf16_round(x).astype(np.float64)
        return x.astype(np.float32).astype(np.float64)


def group_matmul(x, packed, scales, biases, group_size: int, bits: int, dtype: str = "f32",
                 bias=None, relu: bool = False, transpose: bool = True) -> np.ndarray:
    """quantized_matmul in x's dtype, then QuantizedLinearMLX's bias and ReLU, over the rounded
    operands (tolerance reference: MLX's summation order is not knowable): scales and group
    biases cast to x's dtype (lucid/_C/ops/quantized/QuantizedMatmul.cpp:153-164), w_hat =
    c s + b per group (lucid/quantization/_qgemm.py:167-170), y = x w_hat^T (transpose) or
    x w_hat in float64, rounded once to x's dtype ('f16' / 'bf16'; 'f32' keeps the float64
    sum), then fl(y + fl(bias)) and ReLU (lucid/nn/quantized/mlx_linear.py:215-222).  x holds
    values of its dtype."""
    c = group_codes(packed, bits)
    N, K = c.shape
    half = dtype != "f32"

    def rep(a):
        a = np.asarray(a, np.float32)
        return np.repeat((round_to(a, dtype) if half else a.astype(np.float64)).reshape(N, K // group_size),
                         group_size, axis=1)

    w = c * rep(scales)
    if biases is not None:
        w = w + rep(biases)
    y = np.asarray(x, np.float64) @ (w.T if transpose else w)
    if half:
        y = round_to(y, dtype)
    if bias is not None:
        b = np.asarray(bias, np.float32).astype(np.float64)
        y = round_to(y + round_to(b, dtype), dtype) if half else y + b
    if relu:
        y = np.where(y <= 0, 0.0, y)
    return y


# ------------------------------------------- Lucid's multi-pass CPU composition


def set_threads(n: int) -> int:
    return lib().lqo_set_threads(int(n))


def div6_mismatches() -> int:
    """Inputs (of all 2^32 float32) where the GPU activations' fma-corrected division by 6
    differs from the IEEE quotient (0 = the rewrite is exact)."""
    return int(lib().lqo_div6_mismatches())


def lucid_minmax(x: np.ndarray):
    mn = ctypes.c_float()
    mx = ctypes.c_float()
    lib().lqo_lucid_minmax(_ptr(x), x.size, ctypes.byref(mn), ctypes.byref(mx))
    return mn.value, mx.value


def lucid_quantize(x, inv, z, qmin, qmax, q, t0, t1) -> None:
    lib().lqo_lucid_quantize(_ptr(x), x.size, np.float32(inv), np.float32(z), qmin, qmax, _ptr(q),
                             _ptr(t0), _ptr(t1))


def lucid_dequantize(q, s, z, y, t0) -> None:
    lib().lqo_lucid_dequantize(_ptr(q), q.size, np.float32(s), np.float32(z), _ptr(y), _ptr(t0))


# ------------------------------------------------------------- histogram observer


def histc(x: np.ndarray, bins: int, lo: float, hi: float) -> np.ndarray:
    """float32 counts of ``x`` over ``[lo, hi]``: bin trunc((v - lo) / step) in double, the
    top edge in the last bin, values outside the range and NaN skipped."""
    v = np.asarray(x, np.float32).astype(np.float64).ravel()
    step = (hi - lo) / float(bins)
    keep = (v >= lo) & (v <= hi)
    b = ((v[keep] - lo) / step).astype(np.int64)
    b = np.minimum(b, bins - 1)
    return np.bincount(b, minlength=bins).astype(np.float64).astype(np.float32)


def hist_rebin(hist: np.ndarray, old_min: float, old_max: float, new_min: float,
               new_max: float) -> np.ndarray:
    """The stored histogram moved onto ``[new_min, new_max]``: float32 centers and target
    index (each operation rounded to float32), truncation, then an in-order float32
    scatter_add."""
    bins = hist.size
    f = np.float32
    old_w = f((old_max - old_min) / bins)
    new_w = f((new_max - new_min) / bins)
    centers = f(old_min) + (np.arange(bins, dtype=np.float32) + f(0.5)) * old_w
    raw = np.clip((centers - f(new_min)) / new_w, f(0.0), f(bins - 1))
    dst = raw.astype(np.int64)
    out = np.zeros(bins, np.float32)
    for i in range(bins):  # float32 additions in source order
        out[dst[i]] = np.float32(out[dst[i]] + hist[i])
    return out


def histogram_observer(batches, bins: int):
    """(min_val, max_val, histogram) after ``forward`` over ``batches`` (float32 arrays)."""
    mn, mx, hist = np.inf, -np.inf, np.zeros(bins, np.float32)
    for x in batches:
        x = np.asarray(x, np.float32)
        cur_min, cur_max = float(x.min()), float(x.max())
        if mn == np.inf:
            new_min, new_max = cur_min, cur_max
        else:
            new_min, new_max = min(mn, cur_min), max(mx, cur_max)
        lo, hi = new_min, new_max
        if lo == hi:
            lo, hi = cur_min, cur_max
        if not (np.isfinite(lo) and np.isfinite(hi)):
            raise ValueError("histc range is not finite")
        if lo == hi:
            lo, hi = lo - 1.0, hi + 1.0
        h = histc(x, bins, lo, hi)
        if mn == np.inf:
            hist = h
        elif new_min == mn and new_max == mx:
            hist = (h + hist).astype(np.float32)
        else:
            hist = (h + hist_rebin(hist, mn, mx, new_min, new_max)).astype(np.float32)
        mn, mx = float(np.float32(new_min)), float(np.float32(new_max))
    return mn, mx, hist


def hist_clip_search(hist: np.ndarray, lo: float, hi: float, levels: int,
                     quantiles=(0.0, 1e-5, 1e-4, 1e-3, 5e-3, 1e-2)) -> tuple[float, float]:
    """The candidate clip range [quantile(q), quantile(1 - q)] with the least
    sum n_i ((c_i - clip(c_i))^2 + step^2 / 12)."""
    counts = np.asarray(hist, np.float64)
    total = counts.sum()
    if total <= 0.0 or hi <= lo:
        return lo, hi
    bins = counts.size
    width = (hi - lo) / bins
    centers = lo + (np.arange(bins) + 0.5) * width
    cum = np.cumsum(counts)

    def quantile(q: float) -> float:
        idx = np.nonzero(cum >= q * total)[0]
        return float(centers[idx[0]]) if idx.size else float(centers[-1])

    best_err, best = np.inf, (lo, hi)
    nz = counts != 0.0
    for q in quantiles:
        cmin, cmax = quantile(q), quantile(1.0 - q)
        if cmax <= cmin:
            continue
        step = (cmax - cmin) / max(levels, 1)
        cc = np.clip(centers[nz], cmin, cmax)
        err = float(np.sum(counts[nz] * ((centers[nz] - cc) ** 2 + step * step / 12.0)))
        if err < best_err:
            best_err, best = err, (cmin, cmax)
    return best


# ------------------------------------------------------------------- activations

ACT_SIGMOID, ACT_TANH, ACT_HARDSWISH, ACT_HARDSIGMOID, ACT_ELU, ACT_LEAKY_RELU = 0, 1, 2, 3, 4, 5


def activation(x: np.ndarray, op: int, param: float = 0.0) -> np.ndarray:
    """float32 activation with the operation order of Lucid's CPU kernels
    (backend/cpu/methods/Activation.cpp:8-50 sigmoid, 375-400 leaky_relu, 435-460 elu,
    661-686 hard_sigmoid, 726-751 hard_swish; Unary.cpp:165-170 tanh).  Each step rounds to
    float32; ``std::max(t, 0)`` / ``std::min(t, 1)`` are ``t < 0 ? 0 : t`` / ``1 < t ? 1 : t``
    (NaN and -0 pass).  exp / tanh are numpy's float32 functions (the reference's are
    vForce's: these two agree with it to within rounding, not to the bit)."""
    f = np.float32
    x = np.asarray(x, np.float32)
    p = f(param)
    with np.errstate(over="ignore", invalid="ignore"):
        if op == ACT_SIGMOID:
            return (f(1) / (f(1) + np.exp(-x))).astype(np.float32)
        if op == ACT_TANH:
            return np.tanh(x).astype(np.float32)
        if op in (ACT_HARDSWISH, ACT_HARDSIGMOID):
            t = ((x + f(3)) / f(6)).astype(np.float32)
            t = np.where(t < f(0), f(0), t).astype(np.float32)
            t = np.where(f(1) < t, f(1), t).astype(np.float32)
            return (x * t).astype(np.float32) if op == ACT_HARDSWISH else t
        if op == ACT_ELU:
            return np.where(x >= f(0), x, p * (np.exp(x) - f(1))).astype(np.float32)
        if op == ACT_LEAKY_RELU:
            return np.where(x >= f(0), x, p * x).astype(np.float32)
    raise ValueError(f"unknown activation {op}")


# ---------------------------------------------------------------- table lookups

BAG_SUM, BAG_MEAN, BAG_MAX = 0, 1, 2


def embedding_bag(table: np.ndarray, idx: np.ndarray, offsets=None, mode: int = BAG_MEAN,
                  padding_idx: int = -1, include_last_offset: bool = False, bag_len: int = 0,
                  per_sample_weights=None) -> np.ndarray:
    """Pooled lookup over a float32 table (Lucid's CPU kernel, backend/cpu/methods/
    Sequence.cpp:8-93, bags from IndexBounds.h:107-150; per_sample_weights as the composite of
    nn/functional/sparse.py:228-310): each bag walks its indices in order with float32
    additions (sum / mean) or ``v > acc`` replacements from the lowest float (max); padding
    indices skipped and not counted (with weights they add ``v * 0``); mean divides by the
    count when it is positive; an empty max bag is 0.  A bad index raises, as the CPU does."""
    f = np.float32
    table = np.asarray(table, np.float32)
    idx = np.asarray(idx).ravel().astype(np.int64)
    rows, D = table.shape
    n = idx.size
    if offsets is None:
        nb = n // bag_len
        bounds = [(b * bag_len, (b + 1) * bag_len) for b in range(nb)]
    else:
        off = [int(v) for v in np.asarray(offsets).ravel()]
        nb = len(off) - 1 if include_last_offset and off else len(off)
        bounds = [(off[b], off[b + 1] if b + 1 < len(off) else n) for b in range(nb)]
    w = None if per_sample_weights is None else np.asarray(per_sample_weights, np.float32).ravel()
    out = np.zeros((nb, D), np.float32)
    for b, (s, e) in enumerate(bounds):
        acc = np.full(D, np.finfo(np.float32).min if mode == BAG_MAX else 0.0, np.float32)
        count = 0
        for k in range(s, e):
            r = int(idx[k])
            pad = padding_idx >= 0 and r == padding_idx
            if pad and w is None:
                continue
            if not 0 <= r < rows:
                raise IndexError(f"embedding_bag: index {r} out of range")
            v = table[r]
            if w is not None:
                acc = (acc + (v * (f(0) if pad else w[k])).astype(np.float32)).astype(np.float32)
            elif mode == BAG_MAX:
                acc = np.where(v > acc, v, acc).astype(np.float32)
            else:
                acc = (acc + v).astype(np.float32)
            if not pad:
                count += 1
        if mode == BAG_MAX and count == 0:
            acc = np.zeros(D, np.float32)
        if mode == BAG_MEAN and count > 0:
            acc = (acc / f(count)).astype(np.float32)
        out[b] = acc
    return out


# ----------------------------------------------------------------------------- pooling


def pool2d(x: np.ndarray, op: str, kernel=(1, 1), stride=(1, 1), pad=(0, 0), adaptive=None,
           count_include_pad: bool = True) -> np.ndarray:
    """2-D max / average pooling of float32 NCHW ``x`` (backend/cpu/Pool.cpp:27-32, 57-100,
    117-168; adaptive cells nn/functional/_pool_core.py:228-250): max takes the first
    in-window element then any greater one or a NaN; avg sums the in-window elements in
    row-major order in float32 and divides by the window size (padded or not)."""
    x = np.asarray(x, np.float32)
    N, C, H, W = x.shape

    def windows(S, K, st, p, O):
        out = []
        for o in range(O):
            if adaptive is not None:
                lo, hi = (o * S) // O, -((-(o + 1) * S) // O)
                out.append((lo, hi, hi - lo))
            else:
                start = o * st - p
                end = min(start + K, S + p)
                lo, hi = max(start, 0), min(end, S)
                out.append((lo, hi, end - start if count_include_pad else max(hi - lo, 0)))
        return out

    if adaptive is not None:
        OH, OW = adaptive
    else:
        OH = (H + 2 * pad[0] - kernel[0]) // stride[0] + 1
        OW = (W + 2 * pad[1] - kernel[1]) // stride[1] + 1
    wh = windows(H, kernel[0], stride[0], pad[0], OH)
    ww = windows(W, kernel[1], stride[1], pad[1], OW)
    y = np.zeros((N, C, OH, OW), np.float32)
    for oh, (h0, h1, sh) in enumerate(wh):
        for ow, (w0, w1, sw) in enumerate(ww):
            if op == "max":
                best = None
                for h in range(h0, h1):
                    for w in range(w0, w1):
                        v = x[:, :, h, w]
                        if best is None:
                            best = v.copy()
                        else:
                            take = (v > best) | (np.isnan(v) & ~np.isnan(best))
                            best = np.where(take, v, best)
                y[:, :, oh, ow] = best
            else:
                acc = np.zeros((N, C), np.float32)
                for h in range(h0, h1):
                    for w in range(w0, w1):
                        acc = (acc + x[:, :, h, w]).astype(np.float32)
                d = sh * sw
                y[:, :, oh, ow] = (acc / np.float32(d)).astype(np.float32) if d > 0 else 0.0
    return y


# -------------------------------------------------------------------- recurrent layers


def _sig64(x):
    return 1.0 / (1.0 + np.exp(-x))


def rnn_cell(mode: str, gx: np.ndarray, gh: np.ndarray, h: np.ndarray, c=None):
    """One step from the two gate products (float64): ``mode`` RNN_TANH / RNN_RELU / LSTM
    (gates i, f, g, o) / GRU (gates r, z, n) as lucid/nn/modules/rnn.py writes them.  The
    gate width sets H (a projected LSTM's h is narrower and unused here)."""
    H = gx.shape[-1] // {"LSTM": 4, "GRU": 3}.get(mode, 1)
    if mode in ("RNN_TANH", "RNN_RELU"):
        pre = gx + gh
        return (np.tanh(pre) if mode == "RNN_TANH" else np.maximum(pre, 0.0)), None
    if mode == "LSTM":
        g = gx + gh
        i, f, gg, o = _sig64(g[:, :H]), _sig64(g[:, H:2 * H]), np.tanh(g[:, 2 * H:3 * H]), _sig64(g[:, 3 * H:])
        cn = f * c + i * gg
        return o * np.tanh(cn), cn
    r = _sig64(gx[:, :H] + gh[:, :H])
    z = _sig64(gx[:, H:2 * H] + gh[:, H:2 * H])
    n = np.tanh(gx[:, 2 * H:] + r * gh[:, 2 * H:])
    return (1.0 - z) * n + z * h, None


def rnn_forward(mode: str, x: np.ndarray, weights: dict, num_layers: int = 1, bidirectional: bool = False,
                h0=None, c0=None):
    """A multi-layer (bi)directional recurrence over time-major ``x`` [T, B, I] in float64
    with ``weights[name]`` (``weight_ih_l{k}[_reverse]`` ..., biases optional): (output
    [T, B, D R], h_n [L D, B, R], c_n [L D, B, H] or None).  An LSTM with ``weight_hr_l{k}``
    [P, H] is the projected one (lucid/_C/backend/cpu/Lstm.h:90-164): the state carried and
    emitted is h = (o tanh(c)) W_hr^T, R = P wide; otherwise R = H."""
    x = np.asarray(x, np.float64)
    T, B, _ = x.shape
    D = 2 if bidirectional else 1
    R = weights["weight_hh_l0"].shape[1]
    Hc = weights["weight_hh_l0"].shape[0] // {"LSTM": 4, "GRU": 3}.get(mode, 1)
    h_n, c_n = [], []
    inp = x
    for layer in range(num_layers):
        outs = np.zeros((T, B, D * R))
        for d in range(D):
            sfx = f"_l{layer}" + ("_reverse" if d else "")
            w_ih, w_hh = (np.asarray(weights[f"weight_{k}{sfx}"], np.float64) for k in ("ih", "hh"))
            w_hr = weights.get(f"weight_hr{sfx}")
            w_hr = None if w_hr is None else np.asarray(w_hr, np.float64)
            b_ih = np.asarray(weights.get(f"bias_ih{sfx}", np.zeros(w_ih.shape[0])), np.float64)
            b_hh = np.asarray(weights.get(f"bias_hh{sfx}", np.zeros(w_hh.shape[0])), np.float64)
            idx = layer * D + d
            h = np.zeros((B, R)) if h0 is None else np.asarray(h0[idx], np.float64)
            c = np.zeros((B, Hc)) if c0 is None else np.asarray(c0[idx], np.float64)
            for t in (range(T - 1, -1, -1) if d else range(T)):
                h, cn = rnn_cell(mode, inp[t] @ w_ih.T + b_ih, h @ w_hh.T + b_hh, h, c)
                if w_hr is not None:
                    h = h @ w_hr.T
                c = cn if cn is not None else c
                outs[t, :, d * R:(d + 1) * R] = h
            h_n.append(h)
            c_n.append(c)
        inp = outs
    return inp, np.stack(h_n), (np.stack(c_n) if mode == "LSTM" else None)


# ------------------------------------------------------------ transposed convolution


def conv_transpose2d_acc(x, w, za=0, x_u8s8=False, stride=(1, 1), pad=(0, 0), output_padding=(0, 0),
                         dilation=(1, 1), groups=1) -> np.ndarray:
    """Exact int64 accumulators of a transposed convolution, by its direct scatter definition
    (lucid/nn/functional/conv.py conv_transpose2d): y[n, g Cout_g + co, ih s - p + kh d,
    iw s - p + kw d] += (x[n, g Cin_g + ci, ih, iw] - za) w[g Cin_g + ci, co, kh, kw], for codes
    x [N, Cin, H, W] (int8, or the c - 128 form with ``x_u8s8``) and w [Cin, Cout_g, KH, KW]."""
    xv = np.asarray(x, np.int64) + (128 if x_u8s8 else 0) - int(za)
    w = np.asarray(w, np.int64)
    N, Cin, H, W = xv.shape
    _, Cout_g, KH, KW = w.shape
    (sh, sw), (ph, pw), (oph, opw), (dh, dw) = stride, pad, output_padding, dilation
    OH = (H - 1) * sh - 2 * ph + dh * (KH - 1) + oph + 1
    OW = (W - 1) * sw - 2 * pw + dw * (KW - 1) + opw + 1
    cg = Cin // groups
    full = np.zeros((N, groups * Cout_g, (H - 1) * sh + dh * (KH - 1) + 1 + oph,
                     (W - 1) * sw + dw * (KW - 1) + 1 + opw), np.int64)
    for g in range(groups):
        xs = xv[:, g * cg:(g + 1) * cg]
        for kh in range(KH):
            for kw in range(KW):
                contrib = np.einsum("nchw,co->nohw", xs, w[g * cg:(g + 1) * cg, :, kh, kw])
                full[:, g * Cout_g:(g + 1) * Cout_g, kh * dh:kh * dh + (H - 1) * sh + 1:sh,
                     kw * dw:kw * dw + (W - 1) * sw + 1:sw] += contrib
    return full[:, :, ph:ph + OH, pw:pw + OW]


# ------------------------------------------------- float glue of the int8 decoder (config 4)


def layer_norm(x, gamma=None, beta=None, eps: float = 1e-5) -> np.ndarray:
    """(x - mean) / sqrt(var + eps) * gamma + beta over the last axis, biased variance, in
    float64 (nn.LayerNorm's forward)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)
    if beta is not None:
        y = y + np.asarray(beta, np.float64)
    return y


def gelu_tanh(x) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))) in float64 (F.gelu, tanh form)."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def attention(q, k, v, pos0: int, scale: float) -> np.ndarray:
    """Causal attention of q [B, H, n, hd] at positions pos0 .. pos0 + n - 1 over keys /
    values [B, H, T, hd] (T >= pos0 + n; only the first pos0 + n are visible), float64 over
    the given (fp16) values: softmax(scale q k^T, keys <= own position) v -> [B, n, H, hd]."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    B, H, n, hd = q.shape
    T = pos0 + n
    s = np.einsum("bhqd,bhkd->bhqk", q, k[:, :, :T]) * float(np.float32(scale))
    visible = np.arange(T)[None, :] <= (pos0 + np.arange(n))[:, None]
    s = np.where(visible, s, -np.inf)
    s = np.exp(s - s.max(-1, keepdims=True))
    s = s / s.sum(-1, keepdims=True)
    o = np.einsum("bhqk,bhkd->bhqd", s, v[:, :, :T])
    return o.transpose(0, 2, 1, 3)


def embedding_sum(tok_table, pos_table, tokens, pos0: int) -> np.ndarray:
    """tok_table[tokens] + pos_table[pos0 + i] for tokens [B, n] -> [B, n, D] (float32 add)."""
    tokens = np.asarray(tokens)
    n = tokens.shape[-1]
    return (np.asarray(tok_table, np.float32)[tokens] +
            np.asarray(pos_table, np.float32)[pos0:pos0 + n]).astype(np.float32)
