"""``fuse_modules`` and the eval-mode BatchNorm fold (lucid/quantization/fuse_modules.py:62-176,
lucid/nn/utils/fusion.py:28-213).

A run ``[conv, bn?, relu?]`` becomes one module -- the conv with BN folded in, wrapped as
``ConvReLU2d`` when a ReLU follows -- and ``[linear, relu]`` becomes ``LinearReLU``; the
other names of the run become ``Identity`` so the parent's order is unchanged.

BN fold (fusion.py:52-106): ``scale = rsqrt(running_var + eps) * gamma``,
``w' = w * scale[:, None, None, None]``, ``b' = (b - running_mean) * scale + beta``, in
float32.  It is a one-time parameter transform and runs on the host.
"""

from __future__ import annotations

import copy
from typing import Sequence

import numpy as np

from lucid_amd._tensor import tensor
from lucid_amd.nn.module import Module, Parameter


def _get_module(root: Module, dotted: str) -> Module:
    mod = root
    for part in dotted.split("."):
        mod = getattr(mod, part)
    return mod


def _set_module(root: Module, dotted: str, value: Module) -> None:
    parts = dotted.split(".")
    parent = root
    for part in parts[:-1]:
        parent = getattr(parent, part)
    setattr(parent, parts[-1], value)


def fuse_conv_bn_weights(conv_w, conv_b, bn_rm, bn_rv, bn_eps, bn_w, bn_b):
    """Folded ``(weight, bias)`` float32 arrays of a conv (or linear) followed by eval BN."""
    w = np.asarray(conv_w, np.float32)
    C = w.shape[0]
    rm, rv = np.asarray(bn_rm, np.float32), np.asarray(bn_rv, np.float32)
    if rm.shape[0] != C:
        raise ValueError(f"fuse_conv_bn_weights: the BatchNorm has {rm.shape[0]} features but "
                         f"the convolution has {C} output channels")
    scale = (np.float32(1.0) / np.sqrt(rv + np.float32(bn_eps))).astype(np.float32)
    if bn_w is not None:
        scale = (scale * np.asarray(bn_w, np.float32)).astype(np.float32)
    b = np.zeros(C, np.float32) if conv_b is None else np.asarray(conv_b, np.float32)
    fw = (w * scale.reshape((-1,) + (1,) * (w.ndim - 1))).astype(np.float32)
    fb = ((b - rm) * scale).astype(np.float32)
    if bn_b is not None:
        fb = (fb + np.asarray(bn_b, np.float32)).astype(np.float32)
    return fw, fb


def fuse_conv_bn_eval(conv: Module, bn: Module) -> Module:
    """A copy of ``conv`` with eval-mode ``bn`` folded into its weight and bias."""
    if bn.training or conv.training:
        raise AssertionError("Fusion only for eval!")
    fused = copy.deepcopy(conv)
    np_or_none = lambda t: None if t is None else t.numpy()  # noqa: E731
    fw, fb = fuse_conv_bn_weights(conv.weight.numpy(), np_or_none(conv.bias),
                                  bn.running_mean.numpy(), bn.running_var.numpy(), bn.eps,
                                  np_or_none(bn.weight), np_or_none(bn.bias))
    dev = conv.weight.device
    fused.weight = Parameter(tensor(fw, device=dev), conv.weight.requires_grad)
    fused.bias = Parameter(tensor(fb, device=dev),
                           conv.bias.requires_grad if conv.bias is not None else False)
    return fused


def _fuse_run(mods: Sequence[Module]) -> list[Module]:
    import lucid_amd.nn.intrinsic as nni
    from lucid_amd.nn.layers import (BatchNorm1d, BatchNorm2d, BatchNorm3d, Conv1d, Conv2d, Conv3d, Identity, Linear,
                                     ReLU)

    ids = [Identity() for _ in range(len(mods) - 1)]
    first = mods[0]
    runs = ((Conv1d, BatchNorm1d, nni.ConvReLU1d), (Conv2d, BatchNorm2d, nni.ConvReLU2d),
            (Conv3d, BatchNorm3d, nni.ConvReLU3d))
    for conv_t, bn_t, fused_t in runs:
        if type(first) is conv_t:
            conv: Module = first
            rest = list(mods[1:])
            if rest and type(rest[0]) is bn_t:
                conv = fuse_conv_bn_eval(first, rest.pop(0))
            if rest and isinstance(rest[0], ReLU):
                rest.pop(0)
                return [fused_t(conv, ReLU()), *ids]
            return [conv, *ids]
    if isinstance(first, Linear) and len(mods) == 2 and isinstance(mods[1], ReLU):
        return [nni.LinearReLU(first, ReLU()), *ids]
    raise ValueError(f"fuse_modules: unsupported fusion pattern {[type(m).__name__ for m in mods]}")


def fuse_modules(model: Module, modules_to_fuse: Sequence[Sequence[str]],
                 inplace: bool = False) -> Module:
    model = model if inplace else copy.deepcopy(model)
    for group in modules_to_fuse:
        mods = [_get_module(model, name) for name in group]
        for name, repl in zip(group, _fuse_run(mods)):
            _set_module(model, name, repl)
    return model
