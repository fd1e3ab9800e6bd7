"""Float layers a quantized model starts from (the ``nn.Linear`` / ``nn.Conv2d`` /
``nn.ReLU`` / ``nn.BatchNorm2d`` / ``nn.Sequential`` inputs of ``prepare``, ``convert``
and ``quantize_dynamic``, and the activations ``convert`` swaps for quantized ones:
``nn.Sigmoid`` / ``Tanh`` / ``Hardswish`` / ``Hardsigmoid`` / ``ELU`` / ``LeakyReLU``).

Attribute names and parameter shapes follow Lucid's float modules (``weight``
``[out, in]`` / ``[Cout, Cin/groups, kh, kw]``, ``bias``, BatchNorm's ``running_mean`` /
``running_var`` / ``num_batches_tracked``) so ``from_float`` and ``fuse_modules`` read
them unchanged.  Their forward runs the float HIP kernels of ``lucid_amd.nn.functional``
(used for calibration and as the float reference of a quantized model).
"""

from __future__ import annotations

import math
from collections import OrderedDict
from typing import Any, Iterator

import numpy as np

from lucid_amd._tensor import Tensor, tensor
from lucid_amd.nn import functional as F
from lucid_amd.nn.module import Module, Parameter


def _pair(v: Any) -> tuple[int, int]:
    if isinstance(v, (tuple, list)):
        return int(v[0]), int(v[1])
    return int(v), int(v)


_init_rng = np.random.default_rng(0)


def manual_seed(seed: int) -> None:
    """Seed the host generator that initialises float layer parameters."""
    global _init_rng
    _init_rng = np.random.default_rng(seed)


def _uniform(shape: tuple[int, ...], bound: float) -> Tensor:
    return tensor(_init_rng.uniform(-bound, bound, size=shape).astype(np.float32))


class Linear(Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        bound = 1.0 / math.sqrt(in_features) if in_features > 0 else 0.0
        self.weight = Parameter(_uniform((out_features, in_features), bound))
        if bias:
            self.bias = Parameter(_uniform((out_features,), bound))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: Tensor) -> Tensor:
        return F.linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}")


class Conv2d(Module):
    def __init__(self, in_channels: int, out_channels: int, kernel_size: Any, stride: Any = 1,
                 padding: Any = 0, dilation: Any = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros") -> None:
        super().__init__()
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        if isinstance(padding, str):
            self._padding_str = padding
            self.padding = (0, 0)
        else:
            self._padding_str = None
            self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.groups = groups
        self.padding_mode = padding_mode
        fan_in = (in_channels // groups) * self.kernel_size[0] * self.kernel_size[1]
        bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
        self.weight = Parameter(_uniform((out_channels, in_channels // groups, *self.kernel_size),
                                         bound))
        if bias:
            self.bias = Parameter(_uniform((out_channels,), bound))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: Tensor) -> Tensor:
        return F.conv2d(x, self.weight, self.bias, self.stride, self._padding_str or self.padding,
                        self.dilation, self.groups, self.padding_mode)

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, padding={self._padding_str or self.padding}")


def _ntuple(v: Any, n: int, name: str = "") -> tuple[int, ...]:
    from lucid_amd.nn.functional import _ntuple as ntuple

    return ntuple(v, n, name)


class _ConvNd(Module):
    """Float convolution of spatial rank ``_rank`` (lucid/nn/modules/conv.py Conv1d / Conv3d):
    weight [out, in / groups, *kernel]; ``convert`` swaps it for its nn.quantized form."""

    _rank = 2

    def __init__(self, in_channels: int, out_channels: int, kernel_size: Any, stride: Any = 1,
                 padding: Any = 0, dilation: Any = 1, groups: int = 1, bias: bool = True,
                 padding_mode: str = "zeros") -> None:
        super().__init__()
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        n = self._rank
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride = _ntuple(kernel_size, n, "kernel_size"), _ntuple(stride, n, "stride")
        if isinstance(padding, str):
            self._padding_str, self.padding = padding, (0,) * n
        else:
            self._padding_str, self.padding = None, _ntuple(padding, n, "padding")
        self.dilation, self.groups, self.padding_mode = _ntuple(dilation, n, "dilation"), groups, padding_mode
        fan_in = (in_channels // groups) * int(np.prod(self.kernel_size))
        bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
        self.weight = Parameter(_uniform((out_channels, in_channels // groups, *self.kernel_size), bound))
        if bias:
            self.bias = Parameter(_uniform((out_channels,), bound))
        else:
            self.register_parameter("bias", None)

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, padding={self._padding_str or self.padding}")


class Conv1d(_ConvNd):
    _rank = 1

    def forward(self, x: Tensor) -> Tensor:
        return F.conv1d(x, self.weight, self.bias, self.stride, self._padding_str or self.padding,
                        self.dilation, self.groups, self.padding_mode)


class Conv3d(_ConvNd):
    _rank = 3

    def forward(self, x: Tensor) -> Tensor:
        return F.conv3d(x, self.weight, self.bias, self.stride, self._padding_str or self.padding,
                        self.dilation, self.groups, self.padding_mode)


class ReLU(Module):
    def forward(self, x: Tensor) -> Tensor:
        return F.relu(x)


class ConvTranspose2d(Module):
    """Float transposed convolution (lucid/nn/modules/conv.py ConvTranspose2d): weight
    [in, out / groups, kh, kw]; ``convert`` swaps it for ``nn.quantized.ConvTranspose2d``."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size: Any, stride: Any = 1, padding: Any = 0,
                 output_padding: Any = 0, groups: int = 1, bias: bool = True, dilation: Any = 1) -> None:
        super().__init__()
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride = _pair(kernel_size), _pair(stride)
        self.padding, self.output_padding = _pair(padding), _pair(output_padding)
        self.dilation, self.groups = _pair(dilation), groups
        fan_in = (out_channels // groups) * self.kernel_size[0] * self.kernel_size[1]
        bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
        self.weight = Parameter(_uniform((in_channels, out_channels // groups, *self.kernel_size), bound))
        if bias:
            self.bias = Parameter(_uniform((out_channels,), bound))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: Tensor) -> Tensor:
        return F.conv_transpose2d(x, self.weight, self.bias, self.stride, self.padding, self.output_padding,
                                  self.groups, self.dilation)

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}")


class _ConvTransposeNd(Module):
    """Float transposed convolution of spatial rank ``_rank``: weight [in, out / groups, *kernel]."""

    _rank = 1

    def __init__(self, in_channels: int, out_channels: int, kernel_size: Any, stride: Any = 1, padding: Any = 0,
                 output_padding: Any = 0, groups: int = 1, bias: bool = True, dilation: Any = 1) -> None:
        super().__init__()
        if in_channels % groups or out_channels % groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        n = self._rank
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size, self.stride = _ntuple(kernel_size, n, "kernel_size"), _ntuple(stride, n, "stride")
        self.padding, self.output_padding = _ntuple(padding, n, "padding"), _ntuple(output_padding, n, "output_padding")
        self.dilation, self.groups = _ntuple(dilation, n, "dilation"), groups
        fan_in = (out_channels // groups) * int(np.prod(self.kernel_size))
        bound = 1.0 / math.sqrt(fan_in) if fan_in > 0 else 0.0
        self.weight = Parameter(_uniform((in_channels, out_channels // groups, *self.kernel_size), bound))
        if bias:
            self.bias = Parameter(_uniform((out_channels,), bound))
        else:
            self.register_parameter("bias", None)

    def extra_repr(self) -> str:
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}")


class ConvTranspose1d(_ConvTransposeNd):
    _rank = 1

    def forward(self, x: Tensor) -> Tensor:
        return F.conv_transpose1d(x, self.weight, self.bias, self.stride, self.padding, self.output_padding,
                                  self.groups, self.dilation)


class ConvTranspose3d(_ConvTransposeNd):
    _rank = 3

    def forward(self, x: Tensor) -> Tensor:
        return F.conv_transpose3d(x, self.weight, self.bias, self.stride, self.padding, self.output_padding,
                                  self.groups, self.dilation)


class _PaddedTable(Module):
    """A ``[num_embeddings, embedding_dim]`` table, N(0, 1) with the padding row zeroed
    (lucid/nn/modules/sparse.py:_PaddedTable)."""

    def _init_table(self, num_embeddings: int, embedding_dim: int, weight: Tensor | None) -> None:
        if weight is None:
            w = _init_rng.standard_normal((num_embeddings, embedding_dim)).astype(np.float32)
            if self.padding_idx is not None:
                w[self.padding_idx] = 0.0
            weight = tensor(w)
        elif tuple(weight.shape) != (num_embeddings, embedding_dim):
            raise ValueError(f"Shape of weight {tuple(weight.shape)} does not match "
                             f"num_embeddings={num_embeddings} and embedding_dim={embedding_dim}")
        self.weight = Parameter(weight)


class Embedding(_PaddedTable):
    """Float lookup table (lucid/nn/modules/sparse.py:93-346); ``convert`` swaps it for the
    int8 ``nn.quantized.Embedding`` without calibration."""

    def __init__(self, num_embeddings: int, embedding_dim: int, padding_idx: int | None = None,
                 _weight: Tensor | None = None) -> None:
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.padding_idx = F._padding_row(padding_idx, num_embeddings, "Embedding")
        self._init_table(num_embeddings, embedding_dim, _weight)

    def forward(self, input: Tensor) -> Tensor:
        return F.embedding(input, self.weight, self.padding_idx)

    def extra_repr(self) -> str:
        s = f"{self.num_embeddings}, {self.embedding_dim}"
        return s + (f", padding_idx={self.padding_idx}" if self.padding_idx is not None else "")


class EmbeddingBag(_PaddedTable):
    """Float pooled lookup (lucid/nn/modules/sparse.py:349-420): ``mode`` sum / mean / max."""

    def __init__(self, num_embeddings: int, embedding_dim: int, mode: str = "mean",
                 include_last_offset: bool = False, padding_idx: int | None = None,
                 _weight: Tensor | None = None) -> None:
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.mode = mode
        self.include_last_offset = include_last_offset
        self.padding_idx = F._padding_row(padding_idx, num_embeddings, "EmbeddingBag")
        self._init_table(num_embeddings, embedding_dim, _weight)

    def forward(self, input: Tensor, offsets: Tensor | None = None,
                per_sample_weights: Tensor | None = None) -> Tensor:
        return F.embedding_bag(input, self.weight, offsets, self.mode, per_sample_weights,
                               self.include_last_offset, self.padding_idx)

    def extra_repr(self) -> str:
        return f"{self.num_embeddings}, {self.embedding_dim}, mode={self.mode}"


class MaxPool2d(Module):
    def __init__(self, kernel_size: Any, stride: Any = None, padding: Any = 0) -> None:
        super().__init__()
        self.kernel_size = kernel_size
        self.stride = stride if stride is not None else kernel_size
        self.padding = padding

    def forward(self, x: Tensor) -> Tensor:
        return F.max_pool2d(x, self.kernel_size, self.stride, self.padding)

    def extra_repr(self) -> str:
        return f"kernel_size={self.kernel_size}, stride={self.stride}, padding={self.padding}"


class AvgPool2d(Module):
    def __init__(self, kernel_size: Any, stride: Any = None, padding: Any = 0, count_include_pad: bool = True) -> None:
        super().__init__()
        self.kernel_size = kernel_size
        self.stride = stride if stride is not None else kernel_size
        self.padding = padding
        self.count_include_pad = count_include_pad

    def forward(self, x: Tensor) -> Tensor:
        return F.avg_pool2d(x, self.kernel_size, self.stride, self.padding, self.count_include_pad)


class AdaptiveAvgPool2d(Module):
    def __init__(self, output_size: Any) -> None:
        super().__init__()
        self.output_size = output_size

    def forward(self, x: Tensor) -> Tensor:
        return F.adaptive_avg_pool2d(x, self.output_size)

    def extra_repr(self) -> str:
        return f"output_size={self.output_size}"


class Sigmoid(Module):
    def forward(self, x: Tensor) -> Tensor:
        return F.sigmoid(x)


class Tanh(Module):
    def forward(self, x: Tensor) -> Tensor:
        return F.tanh(x)


class Hardswish(Module):
    def forward(self, x: Tensor) -> Tensor:
        return F.hardswish(x)


class Hardsigmoid(Module):
    def forward(self, x: Tensor) -> Tensor:
        return F.hardsigmoid(x)


class ELU(Module):
    def __init__(self, alpha: float = 1.0) -> None:
        super().__init__()
        self.alpha = alpha

    def forward(self, x: Tensor) -> Tensor:
        return F.elu(x, self.alpha)

    def extra_repr(self) -> str:
        return f"alpha={self.alpha}"


class LeakyReLU(Module):
    def __init__(self, negative_slope: float = 0.01) -> None:
        super().__init__()
        self.negative_slope = negative_slope

    def forward(self, x: Tensor) -> Tensor:
        return F.leaky_relu(x, self.negative_slope)

    def extra_repr(self) -> str:
        return f"negative_slope={self.negative_slope}"


class Identity(Module):
    def forward(self, x: Tensor) -> Tensor:
        return x


class Flatten(Module):
    def __init__(self, start_dim: int = 1, end_dim: int = -1) -> None:
        super().__init__()
        self.start_dim = start_dim
        self.end_dim = end_dim

    def forward(self, x: Tensor) -> Tensor:
        shape = list(x.shape)
        s = self.start_dim % len(shape)
        e = self.end_dim % len(shape)
        new = shape[:s] + [int(np.prod(shape[s:e + 1]))] + shape[e + 1:]
        return x.reshape(new)


class BatchNorm2d(Module):
    def __init__(self, num_features: int, eps: float = 1e-5, momentum: float = 0.1,
                 affine: bool = True, track_running_stats: bool = True) -> None:
        super().__init__()
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.affine = affine
        self.track_running_stats = track_running_stats
        if affine:
            self.weight = Parameter(tensor(np.ones(num_features, np.float32)))
            self.bias = Parameter(tensor(np.zeros(num_features, np.float32)))
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)
        self.register_buffer("running_mean", tensor(np.zeros(num_features, np.float32)))
        self.register_buffer("running_var", tensor(np.ones(num_features, np.float32)))
        self.register_buffer("num_batches_tracked", tensor(np.array(0, np.int64)))

    def forward(self, x: Tensor) -> Tensor:
        return F.batch_norm_eval(x, self.running_mean, self.running_var, self.weight, self.bias,
                                 self.eps)

    def extra_repr(self) -> str:
        return f"{self.num_features}, eps={self.eps}"


class BatchNorm1d(BatchNorm2d):
    """Eval BatchNorm over [N, C] or [N, C, L] (the channel axis 1)."""


class BatchNorm3d(BatchNorm2d):
    """Eval BatchNorm over NCDHW."""


class Sequential(Module):
    def __init__(self, *args: Any) -> None:
        super().__init__()
        if len(args) == 1 and isinstance(args[0], OrderedDict):
            for name, m in args[0].items():
                self.add_module(name, m)
        else:
            for i, m in enumerate(args):
                self.add_module(str(i), m)

    def __getitem__(self, idx: int) -> Module:
        mods = list(self._modules.values())
        return mods[idx]

    def __len__(self) -> int:
        return len(self._modules)

    def __iter__(self) -> Iterator[Module]:
        return iter(self._modules.values())

    def forward(self, x: Any) -> Any:
        for m in self._modules.values():
            if m is not None:
                x = m(x)
        return x
