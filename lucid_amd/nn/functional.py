"""Float functional ops on the HIP backend (``F.relu``, ``F.linear``, ...).

Only what a quantized model's float parts need: the activations between quantized
layers and the float model run during calibration.  A code-backed input (the output of
a fake-quantize) is read through its codes where that is exact.
"""

from __future__ import annotations

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32
from lucid_amd.quantization._device import on_device, require_gpu

def _sig():
    import ctypes

    P, I64 = ctypes.c_void_p, ctypes.c_int64
    _C.register_signatures({
        "lq_relu_f32": (ctypes.c_int, [P, P, I64, P]),
        "lq_linear_f32": (ctypes.c_int, [P, I64, P, I64, P, P, I64, I64, I64, I64, P]),
    })


_sig()


def relu(x: Tensor) -> Tensor:
    """``x <= 0 ? 0 : x`` (NaN passes, -0 becomes +0)."""
    require_gpu(x, "relu")
    y = empty(x.shape, float32, "gpu")
    if x.numel():
        _C.call("lq_relu_f32", x.data_ptr(), y.data_ptr(), x.numel(), None)
    return y


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """``x @ weight.T + bias`` in float32 (float model forward)."""
    require_gpu(x, "linear")
    if x.dtype != float32:
        raise TypeError("linear: float32 input expected")
    w = on_device(weight)
    b = on_device(bias) if bias is not None else None
    K = x.shape[-1]
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"linear: input features {K} != weight in_features {w.shape[1]}")
    M = x.numel() // K if K else 0
    y = empty((*x.shape[:-1], N), float32, "gpu")
    if M and N:
        _C.call("lq_linear_f32", x.data_ptr(), K, w.data_ptr(), K,
                b.data_ptr() if b is not None else None, y.data_ptr(), N, M, N, K, None)
    return y


def conv2d(x, weight, bias=None, stride=(1, 1), padding=(0, 0), dilation=(1, 1), groups=1):
    raise NotImplementedError("float conv2d forward is not implemented on the HIP backend yet")


def batch_norm_eval(x, running_mean, running_var, weight, bias, eps):
    raise NotImplementedError("float batch_norm forward is not implemented on the HIP backend yet")
