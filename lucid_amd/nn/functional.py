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


PADDING_MODES = {"zeros": 0, "reflect": 1, "replicate": 2, "circular": 3}


def _pair(v) -> tuple[int, int]:
    if isinstance(v, (tuple, list)):
        return (int(v[0]), int(v[1])) if len(v) > 1 else (int(v[0]), int(v[0]))
    return int(v), int(v)


def conv_padding(padding, kernel: tuple[int, int], dilation: tuple[int, int]) -> tuple[int, int, int, int]:
    """(top, bottom, left, right) of a conv padding: ints, or "valid" / "same" as Lucid resolves
    them (total d * (k - 1), the smaller half before; lucid/nn/functional/_spatial_args.py:141-164)."""
    if isinstance(padding, str):
        if padding == "valid":
            return 0, 0, 0, 0
        if padding != "same":
            raise ValueError(f"unknown padding {padding!r}")
        th, tw = dilation[0] * (kernel[0] - 1), dilation[1] * (kernel[1] - 1)
        return th // 2, th - th // 2, tw // 2, tw - tw // 2
    ph, pw = _pair(padding)
    if ph < 0 or pw < 0:
        raise ValueError("conv2d: padding must be non-negative")
    return ph, ph, pw, pw


def conv2d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0, dilation=1,
           groups: int = 1, padding_mode: str = "zeros") -> Tensor:
    """Float 2-D convolution of NCHW ``x`` (direct kernel, ``lq_conv2d_f32``)."""
    import numpy as np

    require_gpu(x, "conv2d")
    if x.dtype != float32 or x.ndim != 4:
        raise TypeError(f"conv2d: float32 NCHW input expected, got {x.dtype} {x.shape}")
    w = on_device(weight)
    b = on_device(bias) if bias is not None else None
    N, C, H, W = x.shape
    Cout, Cg, KH, KW = w.shape
    if Cg * groups != C:
        raise ValueError(f"conv2d: input has {C} channels, weight expects {Cg} x {groups} groups")
    sh, sw = _pair(stride)
    dh, dw = _pair(dilation)
    pt, pb, pl, pr = conv_padding(padding, (KH, KW), (dh, dw))
    OH = (H + pt + pb - dh * (KH - 1) - 1) // sh + 1
    OW = (W + pl + pr - dw * (KW - 1) - 1) // sw + 1
    if OH < 1 or OW < 1:
        raise ValueError("conv2d: kernel larger than the padded input")
    y = empty((N, Cout, OH, OW), np.float32, "gpu")
    _C.call("lq_conv2d_f32", x.data_ptr(), N, C, H, W, w.data_ptr(),
            b.data_ptr() if b is not None else None, Cout, KH, KW, sh, sw, pt, pb, pl, pr, dh, dw,
            groups, PADDING_MODES[padding_mode], y.data_ptr(), None)
    return y


def batch_norm_eval(x: Tensor, running_mean: Tensor, running_var: Tensor, weight: Tensor | None,
                    bias: Tensor | None, eps: float) -> Tensor:
    """Eval BatchNorm over the channel axis 1: ``((x - mean) * (1 / sqrt(var + eps))) * w + b``."""
    import numpy as np

    require_gpu(x, "batch_norm")
    N, C = x.shape[0], x.shape[1]
    HW = x.numel() // max(N * C, 1)
    y = empty(x.shape, np.float32, "gpu")
    args = [on_device(t) if t is not None else None for t in (running_mean, running_var, weight, bias)]
    _C.call("lq_batch_norm_f32", x.data_ptr(), y.data_ptr(), N, C, HW, args[0].data_ptr(),
            args[1].data_ptr(), args[2].data_ptr() if args[2] is not None else None,
            args[3].data_ptr() if args[3] is not None else None, float(np.float32(eps)), None)
    return y


def _activation(x: Tensor, op: int, param: float, name: str) -> Tensor:
    """One float activation over ``x`` (lq_qact, float32 out); a code-backed input is read
    through its codes."""
    from lucid_amd.nn.quantized.functional_module import _operand

    ptr, xtype, xs, xz = _operand(x, name)
    y = empty(x.shape, float32, "gpu")
    if x.numel():
        _C.call("lq_qact", op, ptr, xtype, xs, xz, x.numel(), param, None, None, 0, 0, _C.F32,
                y.data_ptr(), None)
    return y


def sigmoid(x: Tensor) -> Tensor:
    """``1 / (1 + exp(-x))`` (lucid/nn/functional/activations.py:498-534)."""
    return _activation(x, _C.ACT_SIGMOID, 0.0, "sigmoid")


def tanh(x: Tensor) -> Tensor:
    """``tanh(x)`` (activations.py:537-579)."""
    return _activation(x, _C.ACT_TANH, 0.0, "tanh")


def hardswish(x: Tensor) -> Tensor:
    """``x * min(max((x + 3) / 6, 0), 1)`` (activations.py:399-446)."""
    return _activation(x, _C.ACT_HARDSWISH, 0.0, "hardswish")


def hardsigmoid(x: Tensor) -> Tensor:
    """``min(max((x + 3) / 6, 0), 1)`` (activations.py:449-495)."""
    return _activation(x, _C.ACT_HARDSIGMOID, 0.0, "hardsigmoid")


def elu(x: Tensor, alpha: float = 1.0) -> Tensor:
    """``x >= 0 ? x : alpha * (exp(x) - 1)``, alpha rounded to float32 (activations.py:148-195)."""
    import numpy as np

    return _activation(x, _C.ACT_ELU, float(np.float32(alpha)), "elu")


def leaky_relu(x: Tensor, negative_slope: float = 0.01) -> Tensor:
    """``x >= 0 ? x : negative_slope * x``, the slope rounded to float32 (activations.py:99-145)."""
    import numpy as np

    return _activation(x, _C.ACT_LEAKY_RELU, float(np.float32(negative_slope)), "leaky_relu")
