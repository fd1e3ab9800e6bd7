"""Float functional ops on the HIP backend (``F.relu``, ``F.linear``, ...).

Only what a quantized model's float parts need: the activations between quantized
layers and the float model run during calibration.  A code-backed input (the output of
a fake-quantize) is read through its codes where that is exact.
"""

from __future__ import annotations

import numpy as np

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
    M = int(np.prod(x.shape[:-1], dtype=np.int64))
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
    if isinstance(padding, (tuple, list)) and len(padding) == 4:   # explicit (top, bottom, left, right)
        pads = tuple(int(v) for v in padding)
        if min(pads) < 0:
            raise ValueError("conv2d: padding must be non-negative")
        return pads
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


# ------------------------------------------------------------------- table lookups

_BAG_MODES = {"sum": 0, "mean": 1, "max": 2}


def _strict_index() -> bool:
    """``LUCID_STRICT_INDEX=1``: read GPU indices back and refuse bad ones
    (lucid/nn/functional/_index_checks.py: ``_strict_index``)."""
    import os

    return os.environ.get("LUCID_STRICT_INDEX", "")[:1] not in ("", "0")


def _indices(x: Tensor, rows: int, op: str) -> tuple[Tensor, int]:
    """``x`` as a GPU int32 / int64 index tensor and its type code.  A float ``x`` raises
    ``TypeError``; in strict mode an index outside ``[0, rows)`` raises ``IndexError``
    (_index_checks.py:296-340; otherwise a bad index yields NaN, the reference's GPU policy)."""
    import numpy as np

    if not isinstance(x, Tensor):
        raise TypeError(f"{op}: expected a Tensor of indices, got {type(x).__name__}")
    dt = np.dtype(x.dtype)
    if dt not in (np.int8, np.int16, np.int32, np.int64, np.bool_):
        raise TypeError(f"{op}: indices must be an integer tensor, got {dt}; cast with .to(int64) first")
    if dt not in (np.int32, np.int64):
        x = Tensor._from_numpy(x.numpy().astype(np.int64), "gpu")
    elif x.device != "gpu":
        x = x.to("gpu")
    if _strict_index() and x.numel():
        host = x.numpy().ravel()
        bad = (host < 0) | (host >= rows)
        if bad.any():
            v = int(host[np.argmax(bad)])
            raise IndexError(f"{op}: index {v} is out of range for a table with {rows} entries "
                             f"(valid range [0, {rows - 1}])")
    return x, (_C.I64 if np.dtype(x.dtype) == np.int64 else _C.I32)


def _padding_row(padding_idx, rows: int, op: str):
    """``padding_idx`` as a row of a ``rows``-row table or None (_index_checks.py:390-402)."""
    if padding_idx is None:
        return None
    if not -rows <= padding_idx < rows:
        raise ValueError(f"{op}: padding_idx must be within [-{rows}, {rows}); got {padding_idx}")
    return padding_idx + rows if padding_idx < 0 else padding_idx


def _check_offsets(offsets: Tensor, length: int, op: str):
    """The bag boundaries, read on the host as the reference does on both devices
    (_index_checks.py:410-440): 1-D, within ``[0, length]``, starting at 0, never decreasing."""
    import numpy as np

    if offsets.ndim != 1:
        raise ValueError(f"{op}: offsets must be 1-D, got shape {tuple(offsets.shape)}")
    bounds = [int(v) for v in np.asarray(offsets.numpy()).ravel()]
    for v in bounds:
        if not 0 <= v <= length:
            raise IndexError(f"{op}: offset {v} is out of range for {length} indices "
                             f"(valid range [0, {length}])")
    if bounds and bounds[0] != 0:
        raise ValueError(f"{op}: offsets[0] must be 0, got {bounds[0]}")
    for before, after in zip(bounds, bounds[1:]):
        if after < before:
            raise ValueError(f"{op}: offsets must not decrease, got {after} after {before}")
    arr = np.asarray(bounds, np.int64)
    return Tensor._from_numpy(arr, "gpu"), len(bounds)


def table_lookup(table: int, table_type: int, scale: int | None, zero_point: int | None, rows: int, D: int,
                 input: Tensor, op: str = "embedding") -> Tensor:
    """``lq_embedding`` over a table given by pointers (float32, or int8 codes with row qparams)."""
    import numpy as np

    idx, itype = _indices(input, rows, op)
    y = empty((*input.shape, D), np.float32, "gpu")
    if idx.numel() and D:
        _C.call("lq_embedding", table, table_type, scale, zero_point, rows, D, idx.data_ptr(), itype, idx.numel(),
                y.data_ptr(), None)
    return y


def bag_lookup(table: int, table_type: int, scale: int | None, zero_point: int | None, rows: int, D: int,
               input: Tensor, offsets: Tensor | None, mode: str, per_sample_weights: Tensor | None,
               include_last_offset: bool, padding_idx: int | None, op: str = "embedding_bag") -> Tensor:
    """``lq_embedding_bag`` over a table given by pointers, with the reference's argument rules
    (lucid/nn/functional/sampling.py:489-640, sparse.py:201-334)."""
    import numpy as np

    if mode not in _BAG_MODES:
        raise ValueError(f"embedding_bag: mode must be one of {sorted(_BAG_MODES)}, got {mode!r}")
    pad = _padding_row(padding_idx, rows, op)
    idx, itype = _indices(input, rows, op)
    if per_sample_weights is not None:
        if mode != "sum":
            raise NotImplementedError("embedding_bag: per_sample_weights is only supported for "
                                      f"mode='sum' (got mode={mode!r})")
        if tuple(per_sample_weights.shape) != tuple(input.shape):
            raise ValueError("embedding_bag: per_sample_weights must have the shape of the indices "
                             f"{tuple(input.shape)}, got {tuple(per_sample_weights.shape)}")
        psw = on_device(per_sample_weights)
    else:
        psw = None
    off_ptr, n_off, bag_len = None, 0, 0
    if input.ndim == 2:
        n_bags, bag_len = int(input.shape[0]), int(input.shape[1])
        if bag_len == 0:  # every bag empty
            return Tensor._from_numpy(np.zeros((n_bags, D), np.float32), "gpu")
        include_last_offset = False
    elif input.ndim == 1:
        if offsets is None:
            raise ValueError("embedding_bag: offsets required for 1-D input")
        off_t, n_off = _check_offsets(offsets, int(input.shape[0]), op)
        off_ptr = off_t.data_ptr()
        n_bags = n_off - 1 if include_last_offset and n_off > 0 else n_off
    else:
        raise ValueError(f"embedding_bag: input must be 1-D or 2-D, got {input.ndim}-D")
    y = empty((n_bags, D), np.float32, "gpu")
    if n_bags and D:
        _C.call("lq_embedding_bag", table, table_type, scale, zero_point, rows, D, idx.data_ptr(), itype,
                idx.numel(), off_ptr, _C.I64, n_off, 1 if include_last_offset else 0, bag_len, _BAG_MODES[mode],
                -1 if pad is None else pad, psw.data_ptr() if psw is not None else None, y.data_ptr(), None)
    return y


def embedding(input: Tensor, weight: Tensor, padding_idx: int | None = None) -> Tensor:
    """Rows of the float table ``weight`` (lucid/nn/functional/sparse.py:70-174); padding_idx
    does not mask the forward lookup (Sequence.cpp:538-546)."""
    w = on_device(weight)
    rows, D = int(w.shape[0]), int(w.shape[1])
    _padding_row(padding_idx, rows, "embedding")
    return table_lookup(w.data_ptr(), _C.F32, None, None, rows, D, input)


def embedding_bag(input: Tensor, weight: Tensor, offsets: Tensor | None = None, mode: str = "mean",
                  per_sample_weights: Tensor | None = None, include_last_offset: bool = False,
                  padding_idx: int | None = None) -> Tensor:
    """Pooled rows of the float table ``weight`` (lucid/nn/functional/sampling.py:489-640)."""
    w = on_device(weight)
    return bag_lookup(w.data_ptr(), _C.F32, None, None, int(w.shape[0]), int(w.shape[1]), input, offsets, mode,
                      per_sample_weights, include_last_offset, padding_idx)


# ------------------------------------------------------------------------- pooling


def _pool_input(x: Tensor, op: str):
    """(tensor, pointer, element type, scale ptr, zero-point ptr, QuantSource or None) of a
    4-D pooling input: the codes of a code-backed activation, else float32 storage."""
    from lucid_amd.nn.quantized.functional_module import _operand

    if x.ndim != 4:
        raise ValueError(f"{op}: expected a 4-D (N, C, H, W) input, got {x.ndim}-D")
    ptr, xtype, xs, xz = _operand(x, op)
    return ptr, xtype, xs, xz, x.quant_source if xtype != _C.F32 else None


def max_pool2d(x: Tensor, kernel_size, stride=None, padding=0) -> Tensor:
    """Max over KH x KW windows (lucid/_C/backend/cpu/Pool.cpp:27-100): NaN propagates; a
    code-backed input keeps its grid (the max of the codes is the code of the max)."""
    import numpy as np

    from lucid_amd._tensor import QuantSource

    KH, KW = _pair(kernel_size)
    sh, sw = _pair(stride if stride is not None else kernel_size)
    ph, pw = _pair(padding)
    N, C, H, W = x.shape
    if 2 * ph > KH or 2 * pw > KW:
        raise ValueError("max_pool2d: padding should be at most half of the kernel size")
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    if OH < 1 or OW < 1:
        raise ValueError("max_pool2d: kernel larger than the padded input")
    ptr, xtype, _, _, q = _pool_input(x, "max_pool2d")
    dt = np.float32 if q is None else q.codes.dtype
    y = empty((N, C, OH, OW), dt, "gpu")
    if y.numel():
        _C.call("lq_pool2d", _C.POOL_MAX, ptr, xtype, None, None, N, C, H, W, OH, OW, KH, KW, sh, sw, ph, pw, 0,
                y.data_ptr(), None)
    if q is None:
        return y
    return Tensor._code_backed(QuantSource(y, q.code_type, q.scale, q.zero_point, q.quant_min, q.quant_max), y.shape)


def avg_pool2d(x: Tensor, kernel_size, stride=None, padding=0, count_include_pad: bool = True) -> Tensor:
    """Mean over KH x KW windows (Pool.cpp:117-168), float32 out."""
    KH, KW = _pair(kernel_size)
    sh, sw = _pair(stride if stride is not None else kernel_size)
    ph, pw = _pair(padding)
    N, C, H, W = x.shape
    if 2 * ph > KH or 2 * pw > KW:
        raise ValueError("avg_pool2d: padding should be at most half of the kernel size")
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    if OH < 1 or OW < 1:
        raise ValueError("avg_pool2d: kernel larger than the padded input")
    ptr, xtype, xs, xz, _ = _pool_input(x, "avg_pool2d")
    y = empty((N, C, OH, OW), float32, "gpu")
    if y.numel():
        _C.call("lq_pool2d", _C.POOL_AVG, ptr, xtype, xs, xz, N, C, H, W, OH, OW, KH, KW, sh, sw, ph, pw,
                _C.POOL_COUNT_INCLUDE_PAD if count_include_pad else 0, y.data_ptr(), None)
    return y


def adaptive_avg_pool2d(x: Tensor, output_size) -> Tensor:
    """Mean over the adaptive cells [floor(o S / O), ceil((o + 1) S / O)) of each spatial axis
    (lucid/nn/functional/_pool_core.py:228-250, 407-434), float32 out."""
    N, C, H, W = x.shape
    if isinstance(output_size, (tuple, list)):
        OH, OW = output_size if len(output_size) > 1 else (output_size[0], output_size[0])
    else:
        OH = OW = output_size
    OH = H if OH is None else int(OH)
    OW = W if OW is None else int(OW)
    ptr, xtype, xs, xz, _ = _pool_input(x, "adaptive_avg_pool2d")
    y = empty((N, C, OH, OW), float32, "gpu")
    if y.numel():
        _C.call("lq_pool2d", _C.POOL_AVG, ptr, xtype, xs, xz, N, C, H, W, OH, OW, 1, 1, 1, 1, 0, 0,
                _C.POOL_ADAPTIVE, y.data_ptr(), None)
    return y


# ------------------------------------------------------------ transposed convolution


def convt_geometry(H: int, W: int, kernel, stride, padding, output_padding, dilation):
    """((top, bottom, left, right) padding of the equivalent stride-1 convolution over the
    stride-expanded input, OH, OW) of conv_transpose2d: pad d (k - 1) - p, plus the output
    padding at the bottom / right; OH = (H - 1) s - 2 p + d (k - 1) + op + 1."""
    (KH, KW), (sh, sw), (ph, pw) = _pair(kernel), _pair(stride), _pair(padding)
    (oph, opw), (dh, dw) = _pair(output_padding), _pair(dilation)
    if oph >= max(sh, dh) or opw >= max(sw, dw):
        raise ValueError("conv_transpose2d: output_padding must be smaller than stride or dilation")
    pt, pl = dh * (KH - 1) - ph, dw * (KW - 1) - pw
    if pt < 0 or pl < 0:
        raise NotImplementedError("conv_transpose2d: padding larger than dilation * (kernel - 1) is not supported "
                                  "on the HIP backend")
    OH = (H - 1) * sh - 2 * ph + dh * (KH - 1) + oph + 1
    OW = (W - 1) * sw - 2 * pw + dw * (KW - 1) + opw + 1
    return (pt, pt + oph, pl, pl + opw), OH, OW


def convt_kernel(w, groups: int):
    """A transposed-convolution kernel [Cin, Cout / groups, kh, kw] as the equivalent
    convolution's [Cout, Cin / groups, kh, kw]: channel axes swapped within each group, taps
    flipped (host numpy; codes or floats)."""
    import numpy as np

    Cin, Cout_g, KH, KW = w.shape
    v = w.reshape(groups, Cin // groups, Cout_g, KH, KW).transpose(0, 2, 1, 3, 4)[..., ::-1, ::-1]
    return np.ascontiguousarray(v.reshape(groups * Cout_g, Cin // groups, KH, KW))


def stride_expand(x: Tensor, stride) -> Tensor:
    """``x`` [N, C, H, W] spread by ``stride`` with the zero value in the gaps (the activation
    zero point for a code-backed input, which stays code-backed on its grid)."""
    import numpy as np

    from lucid_amd._tensor import QuantSource

    sh, sw = _pair(stride)
    if (sh, sw) == (1, 1):
        return x
    N, C, H, W = x.shape
    Hu, Wu = (H - 1) * sh + 1, (W - 1) * sw + 1
    q = x.quant_source
    if q is not None and q.code_type in (_C.I8, _C.U8S8):
        y = empty((N, C, Hu, Wu), np.int8, "gpu")
        _C.call("lq_stride_expand", q.codes.data_ptr(), q.code_type, N * C, H, W, sh, sw, q.zero_point.data_ptr(),
                y.data_ptr(), None)
        return Tensor._code_backed(QuantSource(y, q.code_type, q.scale, q.zero_point, q.quant_min, q.quant_max),
                                   y.shape)
    require_gpu(x, "conv_transpose2d")
    y = empty((N, C, Hu, Wu), float32, "gpu")
    _C.call("lq_stride_expand", x.data_ptr(), _C.F32, N * C, H, W, sh, sw, None, y.data_ptr(), None)
    return y


def conv_transpose2d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0,
                     output_padding=0, groups: int = 1, dilation=1) -> Tensor:
    """Float transposed convolution (``weight`` [Cin, Cout / groups, kh, kw]): the stride-1
    convolution of the stride-expanded input with the flipped, channel-swapped kernel
    (the same sums as lucid/nn/functional/conv.py's conv_transpose2d, in another order)."""
    require_gpu(x, "conv_transpose2d")
    if x.ndim != 4 or x.dtype != float32:
        raise TypeError(f"conv_transpose2d: float32 NCHW input expected, got {x.dtype} {x.shape}")
    Cin, _, KH, KW = weight.shape
    if int(x.shape[1]) != Cin:
        raise ValueError(f"conv_transpose2d: input has {int(x.shape[1])} channels, weight expects {Cin}")
    pads, _, _ = convt_geometry(int(x.shape[2]), int(x.shape[3]), (KH, KW), stride, padding, output_padding,
                                dilation)
    w = tensor_of(convt_kernel(weight.numpy(), groups))
    return conv2d(stride_expand(x, stride), w, bias, 1, pads, dilation, groups)


def tensor_of(a):
    """A host array as a GPU tensor."""
    from lucid_amd._tensor import tensor

    return tensor(a, device="gpu")


# ------------------------------------------------------- 1-D and 3-D convolutions
#
# Both run on the 2-D kernels: a 1-D convolution is the 2-D one over a height-1 image; a 3-D
# convolution is the 2-D one over the depth-gathered input (lq_depth_gather: the KD input
# slices an output depth reads, stacked as channels), with the kernel rearranged to
# [Cout, KD C/groups, KH, KW] and the output permuted back to NCDHW (lq_permute_0213).  The
# sums are the 3-D convolution's products, exactly (codes) or in another order (floats).


def _ntuple(v, n: int, name: str = "") -> tuple[int, ...]:
    """``v`` as ``n`` ints, read as Lucid reads a convolution's sizes (nn/modules/
    _conv_common.py:16, nn/functional/_spatial_args.py:28): one int, or a sequence of one, is
    repeated -- except a ``kernel_size``, which must name every axis -- a sequence of ``n``
    is taken as it is, and any other length raises ValueError."""
    if not isinstance(v, (tuple, list)):
        return (int(v),) * n
    vals = tuple(int(x) for x in v)
    if len(vals) == n:
        return vals
    if len(vals) == 1 and name != "kernel_size":
        return vals * n
    what = name or "argument"
    raise ValueError(f"{what} must be an int or a sequence of {n}"
                     f"{'' if name == 'kernel_size' else ' (or of one)'}; got {list(vals)}")


def conv_padding_nd(padding, kernel: tuple[int, ...], dilation: tuple[int, ...]) -> list[tuple[int, int]]:
    """(before, after) per spatial axis: ints (symmetric), or "valid" / "same" as Lucid resolves
    them (total d (k - 1), the smaller half before)."""
    n = len(kernel)
    if isinstance(padding, str):
        if padding == "valid":
            return [(0, 0)] * n
        if padding != "same":
            raise ValueError(f"unknown padding {padding!r}")
        out = []
        for k, d in zip(kernel, dilation):
            t = d * (k - 1)
            out.append((t // 2, t - t // 2))
        return out
    pads = _ntuple(padding, n)
    if min(pads) < 0:
        raise ValueError("conv: padding must be non-negative")
    return [(p, p) for p in pads]


def _grid_of(q, codes):
    from lucid_amd._tensor import QuantSource

    return Tensor._code_backed(QuantSource(codes, q.code_type, q.scale, q.zero_point, q.quant_min, q.quant_max),
                               codes.shape)


def depth_gather(x: Tensor, groups: int, KD: int, OD: int, stride: int, pad: int, dilation: int,
                 expand: int = 1, padding_mode: str = "zeros") -> Tensor:
    """NCDHW ``x`` -> [N OD, KD C, H, W]: for each output depth the KD input slices it reads,
    stacked as channels per group (a code-backed input stays code-backed on its grid)."""
    import numpy as np

    require_gpu(x, "conv3d")
    N, C, D, H, W = (int(s) for s in x.shape)
    shape = (N * OD, KD * C, H, W)
    mode = PADDING_MODES[padding_mode]
    q = x.quant_source
    if q is not None and q.code_type in (_C.I8, _C.U8S8):
        y = empty(shape, np.int8, "gpu")
        _C.call("lq_depth_gather", q.codes.data_ptr(), q.code_type, N, C, D, H * W, groups, KD, OD, stride, pad,
                dilation, expand, mode, q.zero_point.data_ptr(), y.data_ptr(), None)
        return _grid_of(q, y)
    if x.dtype != float32:
        raise TypeError(f"conv3d: float32 input expected, got {x.dtype}")
    y = empty(shape, float32, "gpu")
    _C.call("lq_depth_gather", x.data_ptr(), _C.F32, N, C, D, H * W, groups, KD, OD, stride, pad, dilation, expand,
            mode, None, y.data_ptr(), None)
    return y


def permute_depth(y2: Tensor, N: int, OD: int) -> Tensor:
    """The 2-D convolution's [N OD, Cout, OH, OW] as NCDHW [N, Cout, OD, OH, OW]."""
    import numpy as np

    _, Cout, OH, OW = (int(s) for s in y2.shape)
    shape = (N, Cout, OD, OH, OW)
    q = y2.quant_source
    if q is not None and y2._buf is None:
        codes = empty(shape, np.int8, "gpu")
        _C.call("lq_permute_0213", q.codes.data_ptr(), 1, N, OD, Cout, OH * OW, codes.data_ptr(), None)
        return _grid_of(q, codes)
    y = empty(shape, float32, "gpu")
    _C.call("lq_permute_0213", y2.data_ptr(), 4, N, OD, Cout, OH * OW, y.data_ptr(), None)
    return y


def gathered_kernel(w: Tensor) -> Tensor:
    """A 3-D kernel [Cout, Cg, KD, KH, KW] in the gathered channel order [Cout, KD Cg, KH, KW]
    (float32 or int8, on the GPU)."""
    import numpy as np

    w = w if w.device == "gpu" else w.to("gpu")
    Cout, Cg, KD, KH, KW = (int(s) for s in w.shape)
    out = empty((Cout, KD * Cg, KH, KW), w.dtype, "gpu")
    _C.call("lq_permute_0213", w.data_ptr(), np.dtype(w.dtype).itemsize, Cout, Cg, KD, KH * KW, out.data_ptr(), None)
    return out


def conv3d_geometry(x_shape, kernel, stride, padding, dilation):
    """(depth pads, (top, bottom, left, right), OD) of a 3-D convolution."""
    _, _, D, H, W = x_shape
    (pdf, pdb), (pt, pb), (pl, pr) = conv_padding_nd(padding, kernel, dilation)
    OD = (D + pdf + pdb - dilation[0] * (kernel[0] - 1) - 1) // stride[0] + 1
    if OD < 1:
        raise ValueError("conv3d: kernel larger than the padded input")
    return (pdf, pdb), (pt, pb, pl, pr), OD


def conv3d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0, dilation=1,
           groups: int = 1, padding_mode: str = "zeros") -> Tensor:
    """Float 3-D convolution of NCDHW ``x`` (lucid/nn/functional/conv.py via _convnd, rank 3)."""
    require_gpu(x, "conv3d")
    if x.dtype != float32 or x.ndim != 5:
        raise TypeError(f"conv3d: float32 NCDHW input expected, got {x.dtype} {x.shape}")
    Cout, Cg, KD, KH, KW = (int(s) for s in weight.shape)
    if Cg * groups != int(x.shape[1]):
        raise ValueError(f"conv3d: input has {int(x.shape[1])} channels, weight expects {Cg} x {groups} groups")
    s, d = _ntuple(stride, 3, "stride"), _ntuple(dilation, 3, "dilation")
    (pdf, _), pads, OD = conv3d_geometry(x.shape, (KD, KH, KW), s, padding, d)
    xg = depth_gather(x, groups, KD, OD, s[0], pdf, d[0], 1, padding_mode)
    y2 = conv2d(xg, gathered_kernel(on_device(weight)), bias, s[1:], pads, d[1:], groups, padding_mode)
    return permute_depth(y2, int(x.shape[0]), OD)


def conv1d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0, dilation=1,
           groups: int = 1, padding_mode: str = "zeros") -> Tensor:
    """Float 1-D convolution of NCL ``x``: the 2-D one over a height-1 image."""
    require_gpu(x, "conv1d")
    if x.dtype != float32 or x.ndim != 3:
        raise TypeError(f"conv1d: float32 NCL input expected, got {x.dtype} {x.shape}")
    Cout, Cg, K = (int(s) for s in weight.shape)
    (pl, pr), = conv_padding_nd(padding, (K,), _ntuple(dilation, 1))
    N, C, Lx = (int(s) for s in x.shape)
    y = conv2d(x.reshape(N, C, 1, Lx), on_device(weight).reshape(Cout, Cg, 1, K), bias, (1, _ntuple(stride, 1)[0]),
               (0, 0, pl, pr), (1, _ntuple(dilation, 1)[0]), groups, padding_mode)
    return y.reshape(N, Cout, int(y.shape[3]))


def convt_kernel_nd(w, groups: int):
    """A transposed-convolution kernel [Cin, Cout / groups, *k] as the equivalent convolution's
    [Cout, Cin / groups, *k]: channel axes swapped within each group, every tap axis flipped
    (host numpy; codes or floats)."""
    import numpy as np

    Cin, Cout_g = w.shape[:2]
    ks = w.shape[2:]
    v = w.reshape(groups, Cin // groups, Cout_g, *ks).swapaxes(1, 2)
    v = v[(slice(None),) * 3 + (slice(None, None, -1),) * len(ks)]
    return np.ascontiguousarray(v.reshape(groups * Cout_g, Cin // groups, *ks))


def convt3d_geometry(x_shape, kernel, stride, padding, output_padding, dilation):
    """(depth pad of the equivalent stride-1 convolution, H/W pads, OD, OH, OW) of
    conv_transpose3d; OD = (D - 1) s - 2 p + d (k - 1) + op + 1 per axis."""
    _, _, D, H, W = x_shape
    k, s, p = _ntuple(kernel, 3, "kernel_size"), _ntuple(stride, 3, "stride"), _ntuple(padding, 3, "padding")
    op, d = _ntuple(output_padding, 3), _ntuple(dilation, 3)
    if op[0] >= max(s[0], d[0]):
        raise ValueError("conv_transpose3d: output_padding must be smaller than stride or dilation")
    pd = d[0] * (k[0] - 1) - p[0]
    if pd < 0:
        raise NotImplementedError("conv_transpose3d: padding larger than dilation * (kernel - 1) is not supported "
                                  "on the HIP backend")
    pads, OH, OW = convt_geometry(H, W, k[1:], s[1:], p[1:], op[1:], d[1:])
    OD = (D - 1) * s[0] - 2 * p[0] + d[0] * (k[0] - 1) + op[0] + 1
    return pd, pads, OD, OH, OW


def conv_transpose3d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0,
                     output_padding=0, groups: int = 1, dilation=1) -> Tensor:
    """Float 3-D transposed convolution (``weight`` [Cin, Cout / groups, kd, kh, kw]): H / W
    spread by the stride, the depth expansion folded into the gather, then the stride-1 2-D
    convolution with the flipped, channel-swapped kernel."""
    require_gpu(x, "conv_transpose3d")
    if x.ndim != 5 or x.dtype != float32:
        raise TypeError(f"conv_transpose3d: float32 NCDHW input expected, got {x.dtype} {x.shape}")
    Cin = int(weight.shape[0])
    if int(x.shape[1]) != Cin:
        raise ValueError(f"conv_transpose3d: input has {int(x.shape[1])} channels, weight expects {Cin}")
    k = tuple(int(v) for v in weight.shape[2:])
    s, d = _ntuple(stride, 3, "stride"), _ntuple(dilation, 3, "dilation")
    pd, pads, OD, _, _ = convt3d_geometry(x.shape, k, s, padding, output_padding, d)
    w = gathered_kernel(tensor_of(convt_kernel_nd(weight.numpy(), groups)))
    return convt3d_apply(x, s, pd, d[0], k[0], OD, groups, lambda xg: conv2d(xg, w, bias, 1, pads, d[1:], groups))


def convt3d_apply(x: Tensor, s, pd: int, dd: int, KD: int, OD: int, groups: int, conv) -> Tensor:
    """Expand H / W by the stride, gather the expanded depth axis (channels grouped as the
    equivalent convolution's groups), run ``conv`` (the stride-1 2-D convolution), permute to
    NCDHW."""
    N, C, D, H, W = (int(v) for v in x.shape)
    xe = stride_expand(x.reshape(N, C * D, H, W), s[1:])
    Hu, Wu = int(xe.shape[2]), int(xe.shape[3])
    xg = depth_gather(xe.reshape(N, C, D, Hu, Wu), groups, KD, OD, 1, pd, dd, s[0])
    return permute_depth(conv(xg), N, OD)


def conv_transpose1d(x: Tensor, weight: Tensor, bias: Tensor | None = None, stride=1, padding=0,
                     output_padding=0, groups: int = 1, dilation=1) -> Tensor:
    """Float 1-D transposed convolution: the 2-D one over a height-1 image."""
    require_gpu(x, "conv_transpose1d")
    if x.ndim != 3:
        raise TypeError(f"conv_transpose1d: NCL input expected, got {x.shape}")
    Cin, Cout_g, K = (int(v) for v in weight.shape)
    N, C, Lx = (int(v) for v in x.shape)
    w2 = tensor_of(weight.numpy().reshape(Cin, Cout_g, 1, K))
    y = conv_transpose2d(x.reshape(N, C, 1, Lx), w2, bias, (1, _ntuple(stride, 1)[0]), (0, _ntuple(padding, 1)[0]),
                         (0, _ntuple(output_padding, 1)[0]), groups, (1, _ntuple(dilation, 1)[0]))
    return y.reshape(N, int(y.shape[1]), int(y.shape[3]))
