"""Integer GEMM plumbing behind the quantized Linear layers (``lq_gemm_w8a8``).

Lucid's quantized Linear dequantizes its int8 weight and runs a float ``F.linear`` every
call (lucid/nn/quantized/linear.py:206-215, dynamic/linear.py:85-92).  Here the same
layer runs one W8A8 MFMA GEMM over the integer codes with a fused epilogue:

    acc[m, n] = sum_k (qx[m, k] - zx) * (qw[n, k] - zw[n])           (exact int32)
    y[m, n]   = fl32(fl32(float(acc) * fl32(sx * sw[n])) + bias[n])  [ReLU] [requantize]

:class:`WeightCache` keeps a layer's device-side operands: the codes (Lucid's
``weight_int8 [out, in]``), per-channel scales, the code sums the activation zero point
needs, and -- built on first use -- the MFMA-packed copy the decode path (M <= 128) reads.
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import QuantSource, Tensor, empty
from lucid_amd.quantization._device import on_device, workspace

PACKED_MAX_M = 128


class WeightCache:
    """Device operands of one int8 weight ``[N, K]`` (codes, scales, zero points, sums)."""

    def __init__(self, codes: Tensor, scale: Tensor, zero_point: Tensor | None) -> None:
        if codes.ndim != 2 or codes.dtype != np.int8:
            raise TypeError(f"int8 [out, in] weight codes expected, got {codes.dtype} {codes.shape}")
        self.codes = on_device_codes(codes)
        self.N, self.K = self.codes.shape
        self.scale = _per_row(scale, self.N, "scale")
        self.zero_point = None
        if zero_point is not None:
            z = _per_row(zero_point, self.N, "zero point")
            if np.any(z.numpy() != 0):
                self.zero_point = z
        self.sums = empty((self.N,), np.int32, "gpu")
        if self.N:
            _C.call("lq_row_sums_i8", self.codes.data_ptr(), self.K, self.N, self.K,
                    self.sums.data_ptr(), None)
        self._packed: Tensor | None = None

    def packed(self) -> Tensor | None:
        """The MFMA-packed weight (built once), or None when the shape does not allow it."""
        if self.K % 16:
            return None
        if self._packed is None:
            nbytes = _C.lib().lq_packed_weights_size(self.N, self.K)
            self._packed = empty((max(nbytes, 16),), np.int8, "gpu")
            _C.call("lq_pack_weights_i8", self.codes.data_ptr(), self.K, self.N, self.K,
                    self._packed.data_ptr(), None)
        return self._packed


def _per_row(p: Tensor, N: int, what: str) -> Tensor:
    """A weight qparam as a float32 device vector of N entries (a per-tensor value repeats)."""
    d = on_device(p)
    if d.numel() == 1 and N != 1:
        d = on_device(Tensor._from_numpy(np.full(N, d.item(), np.float32), "cpu"))
    if d.numel() != N:
        raise ValueError(f"weight {what} has {d.numel()} entries for {N} channels")
    return d.reshape(N)


def on_device_codes(codes: Tensor) -> Tensor:
    return codes if codes.device == "gpu" else codes.to("gpu")


def _scalar_or_rows(t: Tensor | None, M: int):
    """(device pointer, stride) of an activation scale: 0-d / one element -> stride 0."""
    if t is None:
        return None, 0, None
    d = on_device(t)
    if d.numel() == 1:
        return d.data_ptr(), 0, d
    if d.numel() != M:
        raise ValueError(f"activation scale has {d.numel()} entries for {M} rows")
    return d.data_ptr(), 1, d


def gemm_w8a8(codes: Tensor, code_type: int, a_scale: Tensor, a_zero_point: Tensor | None,
              w: WeightCache, bias: Tensor | None, out_kind: int, out_scale: Tensor | None = None,
              out_zero_point: Tensor | None = None, qmin: int = 0, qmax: int = 255,
              relu: bool = False) -> Tensor:
    """One W8A8 GEMM over activation codes ``[..., K]`` and a cached weight; returns
    ``[..., N]`` of the output kind's element type (float32 / float16 / codes)."""
    K = codes.shape[-1]
    if K != w.K:
        raise ValueError(f"linear: input features {K} != weight in_features {w.K}")
    M = codes.numel() // K if K else int(np.prod(codes.shape[:-1], dtype=np.int64))
    lead = tuple(codes.shape[:-1])
    out_dt = {_C.OUT_F32: np.float32, _C.OUT_F16: np.float16, _C.OUT_FQ32: np.float32,
              _C.OUT_Q8: np.int8, _C.OUT_QU8S8: np.int8, _C.OUT_QU8: np.uint8,
              _C.OUT_Q16: np.int16, _C.OUT_I32: np.int32}[out_kind]
    y = empty((*lead, w.N), out_dt, "gpu")
    if M == 0 or w.N == 0:
        return y
    flags = (_C.EPI_RELU if relu else 0)
    if code_type == _C.U8S8:
        flags |= _C.EPI_A_U8S8
    elif code_type != _C.I8:
        raise TypeError("activation codes must be int8 (signed grid) or U8S8 (unsigned grid)")
    sa_ptr, sa_stride, _keep_sa = _scalar_or_rows(a_scale, M)
    za = on_device(a_zero_point) if a_zero_point is not None else None
    b = on_device(bias) if bias is not None else None
    os_ = on_device(out_scale) if out_scale is not None else None
    oz = on_device(out_zero_point) if out_zero_point is not None else None
    ws_bytes = _C.lib().lq_gemm_w8a8_workspace_size(M, w.N, K)
    ws = workspace.get(ws_bytes)
    common = (sa_ptr, sa_stride, w.scale.data_ptr(), 1,
              za.data_ptr() if za is not None else None,
              w.zero_point.data_ptr() if w.zero_point is not None else None,
              w.sums.data_ptr(), b.data_ptr() if b is not None else None,
              os_.data_ptr() if os_ is not None else None,
              oz.data_ptr() if oz is not None else None, qmin, qmax, out_kind, flags, ws, ws_bytes,
              None)
    packed = w.packed() if M <= PACKED_MAX_M else None
    if packed is not None and K % 16 == 0:
        _C.call("lq_gemm_w8a8_packed", codes.data_ptr(), K, packed.data_ptr(), y.data_ptr(), w.N, M,
                w.N, K, *common)
    else:
        _C.call("lq_gemm_w8a8", codes.data_ptr(), K, w.codes.data_ptr(), K, y.data_ptr(), w.N, M,
                w.N, K, *common)
    return y


GEMV_PACKED_MAX_M = 16  # lq_gemv_w8_packed's row limit


def gemv_w8(x: Tensor, w: WeightCache, bias: Tensor | None, relu: bool = False) -> Tensor:
    """Weight-only ``x @ dequantize(W)^T + bias`` (ReLU) for a float32 / float16 input
    (``lq_gemv_w8``): the int8 weight is read once, never expanded to float."""
    K = x.shape[-1]
    if K != w.K:
        raise ValueError(f"linear: input features {K} != weight in_features {w.K}")
    M = x.numel() // K if K else int(np.prod(x.shape[:-1], dtype=np.int64))
    y = empty((*x.shape[:-1], w.N), x.dtype, "gpu")
    if M == 0 or w.N == 0:
        return y
    if x.dtype not in (np.float32, np.float16):
        raise TypeError(f"linear: float32 or float16 input expected, got {x.dtype}")
    b = on_device(bias) if bias is not None else None
    xt = _C.F32 if x.dtype == np.float32 else _C.F16
    # 3 <= M <= 16: the MFMA-packed weight (1 KB per wave load); one or two rows read whole
    # weight rows on the VALU kernel of lq_gemv_w8
    use_packed = 3 <= M <= GEMV_PACKED_MAX_M and K >= 16 and x.data_ptr() % 16 == 0
    packed = w.packed() if use_packed else None
    if packed is not None:
        ws_bytes = _C.lib().lq_gemv_w8_packed_workspace_size(M, w.N, K)
        _C.call("lq_gemv_w8_packed", x.data_ptr(), xt, K, packed.data_ptr(), w.scale.data_ptr(),
                w.zero_point.data_ptr() if w.zero_point is not None else None,
                b.data_ptr() if b is not None else None, y.data_ptr(), w.N, M, w.N, K,
                _C.EPI_RELU if relu else 0, workspace.get(ws_bytes), ws_bytes, None)
        return y
    ws_bytes = _C.lib().lq_gemv_w8_workspace_size(M, w.N, K)
    _C.call("lq_gemv_w8", x.data_ptr(), _C.F32 if x.dtype == np.float32 else _C.F16, K,
            w.codes.data_ptr(), K, w.scale.data_ptr(),
            w.zero_point.data_ptr() if w.zero_point is not None else None,
            b.data_ptr() if b is not None else None, y.data_ptr(), w.N, M, w.N, K,
            _C.EPI_RELU if relu else 0, workspace.get(ws_bytes), ws_bytes, None)
    return y


def code_backed_output(codes: Tensor, code_type: int, scale: Tensor, zero_point: Tensor,
                       qmin: int, qmax: int) -> Tensor:
    """Wrap requantized GEMM codes as the float tensor they stand for (the sidecar
    module's fake-quantized output, materialized only when read as floats)."""
    return Tensor._code_backed(QuantSource(codes, code_type, on_device(scale), on_device(zero_point),
                                           qmin, qmax), codes.shape)
