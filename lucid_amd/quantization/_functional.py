"""``quantize`` / ``dequantize`` / ``fake_quantize`` on the HIP backend.

Same signatures and results as lucid/quantization/_functional.py:72-463.  Each
call is one gfx950 kernel launch (lucid_amd/csrc/lq_quant.hip) instead of the
reference's chain of elementwise passes, with the same per-element arithmetic:

* ``quantize``: ``clip(round(x * (1/s)) + z, qmin, qmax)`` cast to the storage dtype,
  the reciprocal multiplied in (``_grid_code``, _functional.py:59-69);
* ``dequantize``: ``(float(q) - z) * s`` (_functional.py:293);
* ``fake_quantize``: the two composed, forward only (_functional.py:326-328).

The reciprocal follows the scale's type as in the reference: a Python float is
inverted in double and rounded once to float32 (``1.0 / s`` is a Python op); a tensor
scale is inverted by a float32 division on the device.
"""

from __future__ import annotations

from typing import Union

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import QuantSource, Tensor, empty, float16, float32
from lucid_amd.quantization._device import CODE_TYPE, ocl, on_device, require_gpu
from lucid_amd.quantization._qscheme import QDtype

_ScaleLike = Union[Tensor, float]
_ZeroPointLike = Union[Tensor, float, int]


def _recip_host(s: float) -> float:
    """fl32(1.0 / s) with the division in double: Lucid's rule for a Python-float scale."""
    return float(np.float32(1.0 / float(s)))


def _per_tensor_args(scale: _ScaleLike, zero_point: _ZeroPointLike, device: str):
    """(d_scale, d_zp, inv_value, scale_value, zp_value, keepalive) for a per-tensor call."""
    keep = []
    if isinstance(scale, Tensor):
        if scale.numel() != 1:
            raise ValueError("per-tensor op got a multi-element scale; pass ch_axis")
        s_t = on_device(scale, device)
        keep.append(s_t)
        d_scale, inv_v, s_v = s_t.data_ptr(), 0.0, 0.0
    else:
        d_scale, inv_v, s_v = None, _recip_host(scale), float(np.float32(scale))
    if isinstance(zero_point, Tensor):
        if zero_point.numel() != 1:
            raise ValueError("per-tensor op got a multi-element zero_point; pass ch_axis")
        z_t = on_device(zero_point, device)
        keep.append(z_t)
        d_zp, z_v = z_t.data_ptr(), 0.0
    else:
        d_zp, z_v = None, float(np.float32(zero_point))
    return d_scale, d_zp, inv_v, s_v, z_v, keep


def _per_channel_args(scale: Tensor, zero_point: _ZeroPointLike, C: int, device: str):
    s_t = on_device(scale, device)
    if s_t.numel() != C:
        raise ValueError(f"per-channel scale has {s_t.numel()} entries for {C} channels")
    keep = [s_t]
    if isinstance(zero_point, Tensor):
        z_t = on_device(zero_point, device)
        if z_t.numel() == 1 and C != 1:
            z_t = on_device(Tensor._from_numpy(np.full(C, z_t.item(), np.float32), "cpu"), device)
        if z_t.numel() != C:
            raise ValueError(f"per-channel zero_point has {z_t.numel()} entries for {C} channels")
        keep.append(z_t)
        return s_t.data_ptr(), z_t.data_ptr(), 0.0, keep
    return s_t.data_ptr(), None, float(np.float32(zero_point)), keep


def _storage_dtype(qdtype: QDtype) -> np.dtype:
    return np.dtype(qdtype.storage)


def quantize(x: Tensor, scale: _ScaleLike, zero_point: _ZeroPointLike, qdtype: QDtype,
             ch_axis: int | None = None) -> Tensor:
    """Integer codes of ``x`` on ``qdtype``'s grid, stored in ``qdtype.storage``."""
    require_gpu(x, "quantize")
    if x.dtype != float32:
        raise TypeError(f"quantize: expected float32 input, got {x.dtype}")
    st = _storage_dtype(qdtype)
    code = CODE_TYPE[st]
    out = empty(x.shape, st, "gpu")
    n = x.numel()
    if n == 0:
        return out
    if ch_axis is not None and isinstance(scale, Tensor):
        outer, C, inner = ocl(x.shape, ch_axis)
        d_s, d_z, z_v, keep = _per_channel_args(scale, zero_point, C, x.device)
        _C.call("lq_quantize_per_channel_f32", x.data_ptr(), out.data_ptr(), outer, C, inner, code,
                d_s, d_z, z_v, qdtype.quant_min, qdtype.quant_max, None)
    else:
        d_s, d_z, inv_v, _s_v, z_v, keep = _per_tensor_args(scale, zero_point, x.device)
        _C.call("lq_quantize_per_tensor_f32", x.data_ptr(), out.data_ptr(), n, code, d_s, d_z,
                inv_v, z_v, qdtype.quant_min, qdtype.quant_max, None)
    del keep
    return out


def dequantize(q: Tensor, scale: _ScaleLike, zero_point: _ZeroPointLike,
               ch_axis: int | None = None, out_dtype=float32) -> Tensor:
    """``(float(q) - z) * s`` as float32 (or float16: the float32 result rounded once)."""
    require_gpu(q, "dequantize")
    code = CODE_TYPE.get(q.dtype)
    if code is None:
        raise TypeError(f"dequantize: unsupported code dtype {q.dtype}")
    out_dtype = np.dtype(out_dtype)
    y_type = _C.F32 if out_dtype == float32 else _C.F16
    if out_dtype not in (float32, float16):
        raise TypeError("dequantize: out_dtype must be float32 or float16")
    out = empty(q.shape, out_dtype, "gpu")
    n = q.numel()
    if n == 0:
        return out
    if ch_axis is not None and isinstance(scale, Tensor):
        outer, C, inner = ocl(q.shape, ch_axis)
        d_s, d_z, z_v, keep = _per_channel_args(scale, zero_point, C, q.device)
        _C.call("lq_dequantize_per_channel", q.data_ptr(), code, out.data_ptr(), y_type, outer, C,
                inner, d_s, d_z, z_v, None)
    else:
        d_s, d_z, _inv, s_v, z_v, keep = _per_tensor_args(scale, zero_point, q.device)
        _C.call("lq_dequantize_per_tensor", q.data_ptr(), code, out.data_ptr(), y_type, n, d_s, d_z,
                s_v, z_v, None)
    del keep
    return out


def fake_quantize(x: Tensor, scale: _ScaleLike, zero_point: _ZeroPointLike, quant_min: int,
                  quant_max: int, ch_axis: int | None = None, return_mask: bool = False):
    """``dequantize(quantize(x))`` in float32; with ``return_mask`` also the straight-through
    mask ``(q_pre >= qmin) * (q_pre <= qmax)`` the reference saves for backward
    (_functional.py:330-332).  Inference only: no autograd graph is recorded."""
    require_gpu(x, "fake_quantize")
    if x.dtype != float32:
        raise TypeError(f"fake_quantize: expected float32 input, got {x.dtype}")
    out = empty(x.shape, float32, "gpu")
    mask = empty(x.shape, float32, "gpu") if return_mask else None
    n = x.numel()
    if n:
        m_ptr = mask.data_ptr() if mask is not None else None
        if ch_axis is not None and isinstance(scale, Tensor):
            outer, C, inner = ocl(x.shape, ch_axis)
            d_s, d_z, z_v, keep = _per_channel_args(scale, zero_point, C, x.device)
            _C.call("lq_fake_quantize_per_channel_f32", x.data_ptr(), out.data_ptr(), outer, C,
                    inner, d_s, d_z, z_v, quant_min, quant_max, m_ptr, None)
        else:
            d_s, d_z, inv_v, s_v, z_v, keep = _per_tensor_args(scale, zero_point, x.device)
            _C.call("lq_fake_quantize_per_tensor_f32", x.data_ptr(), out.data_ptr(), n, d_s, d_z,
                    inv_v, s_v, z_v, quant_min, quant_max, m_ptr, None)
        del keep
    return (out, mask) if return_mask else out


def fake_quantize_to_codes(x: Tensor, scale: Tensor, zero_point: Tensor, quant_min: int,
                           quant_max: int) -> Tensor:
    """Per-tensor fake-quantize whose result is code-backed: the codes are computed (one
    launch) and the float values ``(c - z) * s`` -- bit-identical to ``fake_quantize`` --
    are only materialised if read.  Quantized modules consume the codes directly."""
    require_gpu(x, "fake_quantize")
    s_t = on_device(scale)
    z_t = on_device(zero_point)
    if quant_min >= -128 and quant_max <= 127:
        code_type, st = _C.I8, np.int8
    elif quant_min >= 0 and quant_max <= 255:
        code_type, st = _C.U8S8, np.int8  # MFMA operand form: c - 128
    else:
        return fake_quantize(x, s_t, z_t, quant_min, quant_max)
    codes = empty(x.shape, st, "gpu")
    if x.numel():
        _C.call("lq_quantize_per_tensor_f32", x.data_ptr(), codes.data_ptr(), x.numel(), code_type,
                s_t.data_ptr(), z_t.data_ptr(), 0.0, 0.0, quant_min, quant_max, None)
    return Tensor._code_backed(QuantSource(codes, code_type, s_t, z_t, quant_min, quant_max), x.shape)
