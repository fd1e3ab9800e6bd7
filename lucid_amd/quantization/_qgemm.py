"""Group-wise packed weights and the fused weight-only GEMM (lucid/quantization/_qgemm.py:24-314).

Same three ops and signatures as Lucid's ``_qgemm`` over ``_C_engine.quantized``
(lucid/_C/bindings/bind_quantized.cpp:17-27), on the HIP kernels of
lucid_amd/csrc/lq_wo.hip:

* ``quantize(w, group_size, bits)`` -> ``(packed int32 [N, K*bits/32], scales [N, K/gs],
  biases [N, K/gs])``: per group ``s = (max - min) / (2^bits - 1)``, ``b = min``,
  ``c = clip(round((w - b) / s), 0, 2^bits - 1)``, packed 32/bits codes per word, little end
  first (``lq_group_quantize_f32``);
* ``dequantize(...)`` -> ``c * s + b`` as float32 (``lq_group_dequantize_f32``);
* ``quantized_matmul(x, ...)`` -> ``x @ w_hat^T`` (``transpose=True``) or ``x @ w_hat``
  (``transpose=False``) in x's dtype (``lq_group_matmul``);
* ``quantized_matmul_backward(dy, ...)`` -> the input gradient of ``quantized_matmul``, the
  product against the dequantized weight in the other orientation (QLoRA's dX,
  ``QuantizedMatmulBackward::apply``, lucid/_C/ops/quantized/QuantizedMatmul.cpp:73-90).

Like Lucid's (Metal-only) ops these require device tensors.  The exact scale / rounding /
pack order of MLX 0.32.3, which Lucid calls, is not visible from the reference: these ops
follow the formula Lucid documents (_qgemm.py:84-97, 167-170).
"""

from __future__ import annotations

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, bfloat16, empty, float16, float32
from lucid_amd.quantization._device import on_device, require_gpu, workspace

_GROUP_SIZES = (32, 64, 128)


def is_available() -> bool:
    """True when the group-wise kernels are loadable and a GPU is visible."""
    import lucid_amd.backends as backends

    return backends.quantized.available


def _check(group_size: int, bits: int, K: int, op: str) -> None:
    if group_size not in _GROUP_SIZES:
        raise ValueError(f"{op}: group_size must be one of {_GROUP_SIZES}, got {group_size}")
    if bits not in (4, 8):
        raise ValueError(f"{op}: bits must be 4 or 8, got {bits}")
    if K % group_size:
        raise ValueError(f"{op}: the quantized dimension {K} is not a multiple of group_size "
                         f"{group_size}")


def quantize(w: Tensor, group_size: int = 64, bits: int = 8) -> tuple[Tensor, Tensor, Tensor]:
    """Group-wise quantize a float weight ``[N, K]`` along K."""
    require_gpu(w, "quantized.quantize")
    if w.dtype != float32 or w.ndim != 2:
        raise TypeError(f"quantized.quantize: float32 [out, in] weight expected, got {w.dtype} "
                        f"{w.shape}")
    N, K = w.shape
    _check(group_size, bits, K, "quantized.quantize")
    packed = empty((N, K * bits // 32), np.int32, "gpu")
    scales = empty((N, K // group_size), float32, "gpu")
    biases = empty((N, K // group_size), float32, "gpu")
    if N and K:
        _C.call("lq_group_quantize_f32", w.data_ptr(), N, K, group_size, bits, packed.data_ptr(),
                scales.data_ptr(), biases.data_ptr(), None)
    return packed, scales, biases


def _unpacked_k(wq: Tensor, bits: int) -> int:
    return wq.shape[-1] * 32 // bits


def _check_packed(wq: Tensor, scales: Tensor, biases: Tensor | None, group_size: int, bits: int,
                  op: str) -> tuple[int, int]:
    """Validate the packed operands on the host, before any launch: the kernels index
    ``scales[n * (K / group_size) + k / group_size]``, so a scale table of another shape (a
    group size other than the one it was built with) would be read past its end.  MLX, which
    Lucid calls, rejects such operands too.  Returns (N, K)."""
    if wq.ndim != 2 or wq.dtype not in (np.int32, np.uint32):
        raise TypeError(f"{op}: packed weight must be a 2-D int32 / uint32 tensor, got {wq.dtype} "
                        f"{wq.shape}")
    N, K = wq.shape[0], _unpacked_k(wq, bits)
    _check(group_size, bits, K, op)
    want = (N, K // group_size)
    for name, t in (("scales", scales), ("biases", biases)):
        if t is None:
            continue
        if tuple(t.shape) != want:
            raise ValueError(f"{op}: {name} must be {want} for a {N} x {K} weight with "
                             f"group_size {group_size}, got {tuple(t.shape)}")
    return N, K


def dequantize(wq: Tensor, scales: Tensor, biases: Tensor | None, group_size: int = 64,
               bits: int = 8) -> Tensor:
    """``c * s + b`` as a float32 ``[N, K]`` weight."""
    N, K = _check_packed(wq, scales, biases, group_size, bits, "quantized.dequantize")
    require_gpu(wq, "quantized.dequantize")
    s = on_device(scales)
    b = on_device(biases) if biases is not None else None
    out = empty((N, K), float32, "gpu")
    if N and K:
        _C.call("lq_group_dequantize_f32", wq.data_ptr(), s.data_ptr(),
                b.data_ptr() if b is not None else None, N, K, group_size, bits, out.data_ptr(),
                None)
    return out


def quantized_matmul(x: Tensor, wq: Tensor, scales: Tensor, biases: Tensor | None,
                     transpose: bool = True, group_size: int = 64, bits: int = 8,
                     bias: Tensor | None = None, relu: bool = False) -> Tensor:
    """``x @ w_hat^T`` (``[..., K] -> [..., N]``) or, with ``transpose=False``, ``x @ w_hat``
    (``[..., N] -> [..., K]``), in x's dtype (float32, float16 or bfloat16), for the packed
    ``w_hat [N, K]``.

    ``bias`` (length of the output features) / ``relu`` fuse the layer epilogue of
    ``QuantizedLinearMLX`` into the kernel.

    Dtypes follow Lucid (QuantizedMatmul.cpp:153-164, mlx_linear.py:215-222): the scales,
    group biases and ``bias`` are rounded to x's dtype, the product is x's dtype and the bias
    is added in that dtype.  A bfloat16 x is widened to float32 (exact), multiplied with the
    bfloat16 rounding rule (``lq_group_matmul``'s ``LQ_EPI_ROUND_BF16``) and the bfloat16-valued
    result narrowed back (exact): three launches on one stream.
    """
    if x.dtype not in (float32, float16, bfloat16):
        raise TypeError(f"quantized_matmul: float32, float16 or bfloat16 input expected, got {x.dtype}")
    N, K = _check_packed(wq, scales, biases, group_size, bits, "quantized_matmul")
    d_in, d_out = (K, N) if transpose else (N, K)
    if x.shape[-1] != d_in:
        raise ValueError(f"quantized_matmul: input features {x.shape[-1]} != the weight's "
                         f"{'K' if transpose else 'N'} {d_in}")
    if bias is not None and (bias.numel() != d_out or bias.dtype != float32):
        raise ValueError(f"quantized_matmul: bias must be float32 of {d_out} output features, got "
                         f"{bias.dtype} of {bias.numel()}")
    require_gpu(x, "quantized.quantized_matmul")
    require_gpu(wq, "quantized.quantized_matmul")
    M = int(np.prod(x.shape[:-1], dtype=np.int64))
    s = on_device(scales)
    b = on_device(biases) if biases is not None else None
    lb = on_device(bias) if bias is not None else None
    bf16 = x.dtype == bfloat16
    xk = x.to(dtype=float32) if bf16 else x
    y = empty((*x.shape[:-1], d_out), float32 if bf16 else x.dtype, "gpu")
    if M and d_out:
        ws_bytes = _C.lib().lq_group_matmul_workspace_size(M, N, K, group_size) if transpose else 0
        flags = (_C.EPI_RELU if relu else 0) | (_C.EPI_ROUND_BF16 if bf16 else 0)
        _C.call("lq_group_matmul", xk.data_ptr(), _C.F32 if xk.dtype == float32 else _C.F16, d_in,
                wq.data_ptr(), s.data_ptr(), b.data_ptr() if b is not None else None,
                lb.data_ptr() if lb is not None else None, y.data_ptr(), d_out, M, N, K, group_size,
                bits, 1 if transpose else 0, flags, workspace.get(ws_bytes), ws_bytes, None)
    return y.to(dtype=bfloat16) if bf16 else y


def quantized_matmul_backward(dy: Tensor, wq: Tensor, scales: Tensor, biases: Tensor | None,
                              transpose: bool = True, group_size: int = 64, bits: int = 8) -> Tensor:
    """The input gradient of ``quantized_matmul(x, wq, scales, biases, transpose, ...)``:
    ``dX = dY @ dequant(W)`` for ``transpose=True``, ``dY @ dequant(W)^T`` otherwise, in dY's
    dtype (QuantizedMatmulBackward::apply, lucid/_C/ops/quantized/QuantizedMatmul.cpp:73-90;
    the weight, scales and biases are frozen, so dX is the only gradient).  Computed by the
    fused product in the other orientation, without forming the dequantized weight.
    """
    return quantized_matmul(dy, wq, scales, biases, transpose=not transpose, group_size=group_size,
                            bits=bits)
