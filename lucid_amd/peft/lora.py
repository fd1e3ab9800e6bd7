"""LoRA adapters over the quantized linears (QLoRA) and the float ``Linear``
(lucid/peft/tuners/lora/_layer.py:115-1046, _weight_site.py:162-243, _config.py:270-279).

A LoRA layer keeps the wrapped module as ``base_layer`` (frozen, untouched) and, per adapter
name, two float factors ``lora_A`` ``[r, in]`` and ``lora_B`` ``[out, r]`` (``nn.Linear``
modules, ``lora_B`` with a bias when ``lora_bias``), so a state dict reads
``<layer>.lora_A.<adapter>.weight`` as Lucid's does.  The forward pass is
``y = base(x) + s * B(A(x))`` with ``s = lora_alpha / r`` (``/ sqrt(r)`` with ``use_rslora``):
the base layer's own path (the int8 / group-wise GEMM for a quantized base), the two factor
products on the float GEMM, and the update added by one kernel in Lucid's order
(``lq_add_scaled_f32``: the product times ``s``, rounded, then added).

Merging folds ``s B A`` into the base weight.  A float ``Linear`` adds it in place (unmerge
subtracts it).  A quantized base (``nnq.Linear``, ``nnqd.Linear``, ``QuantizedLinearMLX``) is
dequantized, the delta added, and the sum requantized the way Lucid's weight sites do: int8
weights by a per-channel symmetric ``qint8`` min/max observer along ``weight_ch_axis``,
group-wise weights by the group quantizer at the layer's ``group_size`` / ``bits``; the
quantized buffers from before the first merge are kept, and ``unmerge`` restores exactly
those (no requantization drift).  Everything runs on the GPU.

This backend has no autograd: the adapters are for inference with trained factors (loaded
through ``load_state_dict``) and for merging.  Dropout is the identity in eval mode; a layer
in training mode with ``lora_dropout > 0`` raises.
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass, field

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import Tensor, empty, float32, tensor
from lucid_amd.nn import functional as F
from lucid_amd.nn.layers import Linear as FloatLinear
from lucid_amd.nn.module import Module, Parameter
from lucid_amd.quantization._device import on_device, require_gpu


def _check_rank(value: object) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"`r` must be an int, got {value!r}")
    if value <= 0:
        raise ValueError(f"`r` should be a positive integer value but the value passed is {value}")
    return value


def _check_number(name: str, value: object) -> float:
    if isinstance(value, bool) or not isinstance(value, (int, float)) or not math.isfinite(float(value)):
        raise TypeError(f"`{name}` must be a finite number, got {value!r}")
    return float(value)


@dataclass
class LoraConfig:
    """The LoRA settings of ``lucid.peft.LoraConfig`` this backend honours
    (lucid/peft/tuners/lora/_config.py:270-279; validation _config.py:196-244)."""

    r: int = 8
    target_modules: str | list[str] | set[str] | None = None
    lora_alpha: float = 8
    lora_dropout: float = 0.0
    use_rslora: bool = False
    lora_bias: bool = False
    init_lora_weights: bool | str = True
    peft_type: str = field(default="LORA", init=False)

    def __post_init__(self) -> None:
        _check_rank(self.r)
        self.lora_alpha = _check_number("lora_alpha", self.lora_alpha)
        p = _check_number("lora_dropout", self.lora_dropout)
        if not 0.0 <= p < 1.0:
            raise ValueError(f"`lora_dropout` must lie in [0, 1), got {p}")
        if self.init_lora_weights not in (True, False, "gaussian"):
            raise ValueError(f"init_lora_weights {self.init_lora_weights!r} is not supported here "
                             "(True, False or 'gaussian')")
        if isinstance(self.target_modules, (list, tuple)):
            self.target_modules = set(self.target_modules)

    @property
    def scaling(self) -> float:
        return self.lora_alpha / (math.sqrt(self.r) if self.use_rslora else self.r)

    def matches(self, key: str) -> bool:
        """Whether the module at path ``key`` is a target: a string is matched whole as a regular
        expression, a collection by name or dotted suffix (lucid/peft/_targeting.py:35,88-93)."""
        t = self.target_modules
        if t is None:
            raise ValueError("LoraConfig.target_modules must name the modules to adapt")
        if isinstance(t, str):
            return re.fullmatch(t, key) is not None
        return any(key == name or key.endswith(f".{name}") for name in t)


class _Table(Module):
    """Per-adapter modules by name (Lucid's ``ModuleDict`` of factors)."""

    def __getitem__(self, name: str) -> Module:
        return self._modules[name]

    def __contains__(self, name: str) -> bool:
        return name in self._modules

    def keys(self):
        return list(self._modules)


def _gpu(t: Tensor) -> Tensor:
    """A code buffer on the GPU, its dtype kept."""
    return t if t.device == "gpu" else t.to("gpu")


def _quantized_types() -> tuple[type, ...]:
    import lucid_amd.nn.quantized as nnq
    import lucid_amd.nn.quantized.dynamic as nnqd

    return (nnq.QuantizedLinearMLX, nnq.Linear, nnqd.Linear)


class Linear(Module):
    """A float ``Linear`` with LoRA updates: ``y = W x + b + sum_a s_a B_a A_a x``
    (lucid/peft/tuners/lora/_layer.py:822-989)."""

    def __init__(self, base_layer: Module, adapter_name: str, config: LoraConfig) -> None:
        super().__init__()
        self.base_layer = base_layer
        self.lora_A = _Table()
        self.lora_B = _Table()
        self._specs: dict[str, tuple[int, float, float, bool, float]] = {}  # r, alpha, s, lora_bias, dropout
        self.merged_adapters: list[str] = []
        self.active_adapter: list[str] = [adapter_name]
        self.disable_adapters = False
        self._saved = None
        self.update_layer(adapter_name, config)

    # --------------------------------------------------------------- shape
    @property
    def in_features(self) -> int:
        return int(self.base_layer.in_features)

    @property
    def out_features(self) -> int:
        return int(self.base_layer.out_features)

    @property
    def merged(self) -> bool:
        return bool(self.merged_adapters)

    def update_layer(self, adapter_name: str, config: LoraConfig) -> None:
        """Create adapter ``adapter_name``: A uniform in +-1/sqrt(in) (Lucid's Kaiming default),
        or N(0, 1/r) with ``init_lora_weights="gaussian"``; B zero, so the layer starts as its
        base; ``init_lora_weights=False`` leaves B random too."""
        if adapter_name in self._specs:
            raise ValueError(f"adapter {adapter_name!r} already exists on this layer")
        r = config.r
        a = FloatLinear(self.in_features, r, bias=False)
        b = FloatLinear(r, self.out_features, bias=config.lora_bias)
        if config.init_lora_weights == "gaussian":
            rng = np.random.default_rng()
            a.weight = Parameter(tensor(rng.normal(0.0, 1.0 / r, (r, self.in_features)).astype(np.float32)))
        if config.init_lora_weights is not False:
            b.weight = Parameter(tensor(np.zeros((self.out_features, r), np.float32)))
            if b.bias is not None:
                b.bias = Parameter(tensor(np.zeros(self.out_features, np.float32)))
        self.lora_A.add_module(adapter_name, a)
        self.lora_B.add_module(adapter_name, b)
        self._specs[adapter_name] = (r, config.lora_alpha, config.scaling, config.lora_bias, config.lora_dropout)
        for p in self.base_layer.parameters():
            p.requires_grad = False

    def set_adapter(self, names: str | list[str]) -> None:
        names = [names] if isinstance(names, str) else list(names)
        for n in names:
            if n not in self._specs:
                raise ValueError(f"adapter {n!r} not found on this layer")
        self.active_adapter = names

    def scaling(self, adapter: str) -> float:
        return self._specs[adapter][2]

    # ------------------------------------------------------------- forward
    def _update(self, adapter: str, x: Tensor) -> Tensor:
        """B(A(x)) in float32 (the second factor's bias included), before the scale."""
        if self.training and self._specs[adapter][4] > 0:
            raise NotImplementedError("LoRA dropout in training mode needs autograd, which this backend does "
                                      "not run; call .eval() for inference")
        a, b = self.lora_A[adapter], self.lora_B[adapter]
        return F.linear(F.linear(x, a.weight), b.weight, b.bias)

    def forward(self, x: Tensor) -> Tensor:
        result = self.base_layer(x)
        if self.disable_adapters:
            return result
        applied = [n for n in self.active_adapter if n in self._specs and n not in self.merged_adapters]
        if not applied:
            return result
        require_gpu(result, "LoRA layer")
        if x.dtype != float32 or result.dtype != float32:
            raise TypeError("LoRA layer: float32 input and base output expected")
        out = result
        for adapter in applied:
            u = self._update(adapter, x)
            y = empty(out.shape, float32, "gpu")
            _C.call("lq_add_scaled_f32", out.data_ptr(), u.data_ptr(), np.float32(self.scaling(adapter)),
                    y.data_ptr(), out.numel(), None)
            out = y
        return out

    # -------------------------------------------------------------- merging
    def get_delta_weight(self, adapter: str) -> Tensor:
        """``s * (B @ A)`` as float32 [out, in], each product and the scale rounded once."""
        a = on_device(self.lora_A[adapter].weight)
        b = on_device(self.lora_B[adapter].weight)
        r = self._specs[adapter][0]
        at = empty((self.in_features, r), float32, "gpu")
        _C.call("lq_transpose_f32", a.data_ptr(), r, self.in_features, at.data_ptr(), None)
        ba = F.linear(b, at)  # [out, r] @ [r, in]
        zero = tensor(np.zeros(ba.shape, np.float32), device="gpu")
        delta = empty(ba.shape, float32, "gpu")
        _C.call("lq_add_scaled_f32", zero.data_ptr(), ba.data_ptr(), np.float32(self.scaling(adapter)),
                delta.data_ptr(), ba.numel(), None)
        return delta

    def _shift_rows(self, weight: Tensor, adapter: str, sign: float) -> Tensor:
        """``weight + sign * s (B @ A)`` as float32 (Lucid's ``_added``)."""
        a = on_device(self.lora_A[adapter].weight)
        b = on_device(self.lora_B[adapter].weight)
        r = self._specs[adapter][0]
        at = empty((self.in_features, r), float32, "gpu")
        _C.call("lq_transpose_f32", a.data_ptr(), r, self.in_features, at.data_ptr(), None)
        ba = F.linear(b, at)
        w = on_device(weight)
        out = empty(w.shape, float32, "gpu")
        _C.call("lq_add_scaled_f32", w.data_ptr(), ba.data_ptr(), np.float32(sign * self.scaling(adapter)),
                out.data_ptr(), w.numel(), None)
        return out

    def _bias_shift(self, adapter: str, sign: float) -> None:
        b = self.lora_B[adapter].bias
        if b is None:
            return
        base_bias = self.base_layer.bias
        if base_bias is None:
            raise RuntimeError("the base layer has no bias to merge lora_bias into")
        cur = on_device(base_bias)
        out = empty(cur.shape, float32, "gpu")
        _C.call("lq_add_scaled_f32", cur.data_ptr(), on_device(b).data_ptr(), np.float32(sign * self.scaling(adapter)),
                out.data_ptr(), cur.numel(), None)
        self._write_bias(out)

    def _write_bias(self, value: Tensor) -> None:
        if isinstance(self.base_layer.bias, Parameter):
            self.base_layer.bias = Parameter(value, self.base_layer.bias.requires_grad)
        else:
            self.base_layer.register_buffer("bias", value)

    def _read_weight(self) -> Tensor:
        return on_device(self.base_layer.weight)

    def _write_weight(self, value: Tensor) -> None:
        self.base_layer.weight = Parameter(value, False)

    def merge(self, adapter_names: list[str] | None = None) -> None:
        """Fold the active (or named) adapters into the base weight, in order."""
        names = self.active_adapter if adapter_names is None else list(adapter_names)
        for n in names:
            if n not in self._specs:
                raise ValueError(f"adapter {n!r} not found on this layer")
            if n in self.merged_adapters:
                continue
            self._before_first_merge()
            self._write_weight(self._shift_rows(self._read_weight(), n, 1.0))
            self._bias_shift(n, 1.0)
            self.merged_adapters.append(n)

    def _before_first_merge(self) -> None:
        pass

    def unmerge(self) -> None:
        """Take every merged adapter back out (latest first)."""
        for n in reversed(self.merged_adapters):
            self._write_weight(self._shift_rows(self._read_weight(), n, -1.0))
            self._bias_shift(n, -1.0)
        self.merged_adapters = []

    def extra_repr(self) -> str:
        return f"adapters={list(self._specs)}, active={self.active_adapter}, merged={self.merged_adapters}"


class QuantizedLinear(Linear):
    """A quantized linear (``QuantizedLinearMLX``, ``nnq.Linear`` or ``nnqd.Linear``) with float
    LoRA updates (lucid/peft/tuners/lora/_layer.py:992-1046): the base keeps its quantized
    buffers and its own forward path; merging dequantizes, adds ``s B A`` and requantizes as
    Lucid's weight sites do (_weight_site.py:162-243); unmerging restores the buffers saved
    before the first merge."""

    def _is_mlx(self) -> bool:
        import lucid_amd.nn.quantized as nnq

        return isinstance(self.base_layer, nnq.QuantizedLinearMLX)

    def _read_weight(self) -> Tensor:
        from lucid_amd.quantization._functional import dequantize
        from lucid_amd.quantization._qgemm import dequantize as dequantize_mlx

        base = self.base_layer
        if self._is_mlx():
            return dequantize_mlx(_gpu(base.packed_weight), on_device(base.scales), on_device(base.biases),
                                  group_size=base.group_size, bits=base.bits)
        return dequantize(_gpu(base.weight_int8), on_device(base.weight_scale),
                          on_device(base.weight_zero_point), ch_axis=base.weight_ch_axis)

    def _write_weight(self, value: Tensor) -> None:
        from lucid_amd.quantization._functional import quantize
        from lucid_amd.quantization._qgemm import quantize as quantize_mlx
        from lucid_amd.quantization._qscheme import per_channel_symmetric, qint8
        from lucid_amd.quantization.observer import PerChannelMinMaxObserver

        base = self.base_layer
        if self._is_mlx():
            packed, scales, biases = quantize_mlx(value, group_size=base.group_size, bits=base.bits)
            base.register_buffer("packed_weight", packed)
            base.register_buffer("scales", scales)
            base.register_buffer("biases", biases)
            return
        obs = PerChannelMinMaxObserver(ch_axis=base.weight_ch_axis, qscheme=per_channel_symmetric, qdtype=qint8)
        obs(value)
        scale, zero_point = obs.calculate_qparams()
        codes = quantize(value, scale, zero_point, qint8, ch_axis=base.weight_ch_axis)
        base.register_buffer("weight_int8", codes)
        base.register_buffer("weight_scale", scale)
        base.register_buffer("weight_zero_point", zero_point)

    def _before_first_merge(self) -> None:
        if not self.merged_adapters:
            self._saved = {name: buf.clone() for name, buf in self.base_layer._buffers.items()
                           if name != "bias" and buf is not None}

    def unmerge(self) -> None:
        saved = self._saved
        if saved is None:
            return super().unmerge()
        for n in reversed(self.merged_adapters):
            self._bias_shift(n, -1.0)
        for name, buf in saved.items():
            self.base_layer.register_buffer(name, buf)
        self._saved = None
        self.merged_adapters = []


def lora_layer_for(module: Module, adapter_name: str, config: LoraConfig) -> Linear | None:
    """The LoRA layer that adapts ``module``, or None when this backend has none for its type."""
    if isinstance(module, _quantized_types()):
        return QuantizedLinear(module, adapter_name, config)
    if isinstance(module, FloatLinear):
        return Linear(module, adapter_name, config)
    return None
