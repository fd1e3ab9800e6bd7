"""Dispatch registration: ``prepare`` / ``convert`` / ``quantize_dynamic``
(lucid/quantization/_quantize.py:46-778).

* ``prepare`` resolves every module's ``QConfig``, gives each observed type (Linear,
  Conv2d, the fused blocks, ``QuantStub``) an ``activation_post_process`` observer fed by a
  forward hook (_quantize.py:199-304);
* ``convert`` swaps each calibrated module for its quantized form through the
  ``type -> from_float`` mapping (``_quant_mapping``, _quantize.py:74-121), depth first, in
  place of the child so a ``Sequential`` keeps its order (_quantize.py:759-778);
* ``quantize_dynamic`` swaps ``Linear`` for the dynamic int8 layer per ``qconfig_spec``
  (_quantize.py:429-620).

With ``lucid_amd.backends.quantized.use_mlx()`` the Linear family is routed to the
group-wise weight-only layer instead, when ``in_features`` is divisible by a supported
group size (``_mlx_group_size``: 64, then 128, then 32; _quantize.py:134-185).
"""

from __future__ import annotations

import copy
import warnings
from typing import Callable

from lucid_amd.nn.module import Module
from lucid_amd.quantization._propagate import (Site, as_mapping, clear_marks, dynamic_rules,
                                               mark, names_a_recipe, plan_sites, weight_dtype)
from lucid_amd.quantization._qscheme import QDtype, qint8
from lucid_amd.quantization.qconfig import QConfig, QConfigMapping, get_default_qconfig_mapping

_FromFloat = Callable[[Module], Module]


def _observed_types() -> tuple[type, ...]:
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.nn.quantized as nnq

    return (nn.Linear, nn.Conv1d, nn.Conv2d, nn.Conv3d, nn.ConvTranspose1d, nn.ConvTranspose2d, nn.ConvTranspose3d,
            nni.ConvReLU1d, nni.ConvReLU2d, nni.ConvReLU3d, nni.LinearReLU, nn.Sigmoid, nn.Hardswish,
            nn.Hardsigmoid, nn.Tanh, nn.ELU, nn.LeakyReLU, nnq.QuantStub, nnq.FloatFunctional)


def _quant_mapping() -> dict[type, _FromFloat]:
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.nn.quantized as nnq

    mapping: dict[type, _FromFloat] = {
        nn.Linear: nnq.Linear.from_float,
        nni.LinearReLU: nnq.LinearReLU.from_float,
        nnq.QuantStub: nnq.Quantize.from_float,
        nnq.DeQuantStub: nnq.DeQuantize.from_float,
        nnq.FloatFunctional: nnq.QFunctional.from_float,
        nn.Sigmoid: nnq.Sigmoid.from_float,
        nn.Hardswish: nnq.Hardswish.from_float,
        nn.Hardsigmoid: nnq.Hardsigmoid.from_float,
        nn.Tanh: nnq.Tanh.from_float,
        nn.ELU: nnq.ELU.from_float,
        nn.LeakyReLU: nnq.LeakyReLU.from_float,
        nn.ConvTranspose1d: nnq.ConvTranspose1d.from_float,
        nn.ConvTranspose2d: nnq.ConvTranspose2d.from_float,
        nn.ConvTranspose3d: nnq.ConvTranspose3d.from_float,
        nn.Conv1d: nnq.Conv1d.from_float,
        nn.Conv3d: nnq.Conv3d.from_float,
        nni.ConvReLU1d: nnq.ConvReLU1d.from_float,
        nni.ConvReLU3d: nnq.ConvReLU3d.from_float,
        nn.Embedding: nnq.Embedding.from_float,
        nn.EmbeddingBag: nnq.EmbeddingBag.from_float,
    }
    if hasattr(nnq, "Conv2d"):
        mapping[nn.Conv2d] = nnq.Conv2d.from_float
        mapping[nni.ConvReLU2d] = nnq.ConvReLU2d.from_float
    return mapping


def _mlx_weight_bits(mod: Module) -> int:
    """Weight bit width (4 / 8) for the group-wise path, from the module's qconfig."""
    qcfg = getattr(mod, "qconfig", None)
    if qcfg is not None:
        bits = getattr(getattr(qcfg.weight(), "qdtype", None), "bits", None)
        if isinstance(bits, int) and bits in (4, 8):
            return bits
    return 8


def _mlx_group_size(in_features: int) -> int | None:
    """Largest supported group size (64, 128, 32 in that order) dividing ``in_features``."""
    for gs in (64, 128, 32):
        if in_features % gs == 0:
            return gs
    return None


def _group_layer():
    import lucid_amd.nn.quantized as nnq

    cls = getattr(nnq, "QuantizedLinearMLX", None)
    if cls is None:
        raise NotImplementedError("the group-wise weight-only Linear is not built into this "
                                  "backend; set lucid_amd.backends.quantized.engine = 'reference'")
    return cls


def _mlx_linear_builder(relu: bool) -> _FromFloat:
    import lucid_amd.nn.quantized as nnq

    dequant = nnq.LinearReLU.from_float if relu else nnq.Linear.from_float

    def build(child: Module) -> Module:
        inner = child[0] if relu else child
        gs = _mlx_group_size(inner.in_features)
        if gs is None:
            return dequant(child)
        return _group_layer().from_float(inner, bits=_mlx_weight_bits(child), group_size=gs,
                                         relu=relu)

    return build


def _mlx_dynamic_builder():
    import lucid_amd.nn.quantized.dynamic as nnqd

    def build(child: Module, dtype: QDtype) -> Module:
        gs = _mlx_group_size(child.in_features)
        if gs is None:
            return nnqd.Linear.from_float(child, dtype)
        return _group_layer().from_float(child, bits=dtype.bits, group_size=gs, relu=False)

    return build


def _observe_outputs(module: Module, observer: Module) -> None:
    """Give ``module`` its activation observer: kept as ``activation_post_process`` (so
    ``convert`` finds the calibrated range) and fed every forward output by a hook."""
    module.activation_post_process = observer
    module.register_forward_hook(lambda _m, _args, output: observer(output))


def prepare(model: Module, qconfig: QConfig | QConfigMapping | None = None,
            inplace: bool = False) -> Module:
    """Attach activation observers to every quantizable module (static PTQ).

    Each module's recipe is resolved (own ``.qconfig`` > name rule > type rule > parent;
    the stock default only for models the user has not configured) and written onto it as
    ``.qconfig``; each observed type with a recipe gets its activation observer."""
    mapping, stock = as_mapping(qconfig, get_default_qconfig_mapping)
    model = model if inplace else copy.deepcopy(model)
    model.eval()
    sites = plan_sites(model, mapping, stock_default=stock)
    mark(sites)
    observed = _observed_types()
    targets = [site for site in sites if site.qconfig is not None and isinstance(site.module, observed)]
    for site in targets:
        _observe_outputs(site.module, site.qconfig.activation())
    if not targets:
        warnings.warn("prepare(): the QConfigMapping matched no quantizable modules -- "
                      "convert() will leave this model unchanged.", stacklevel=2)
    return model


def _convert_recursive(module: Module, mapping: dict, always: tuple) -> None:
    for name, child in list(module.named_children()):
        build = mapping.get(type(child))
        excluded = "qconfig" in child.__dict__ and child.__dict__["qconfig"] is None
        convertible = build is not None and (
            (isinstance(child, always) and not excluded)
            or "activation_post_process" in child._modules
        )
        if convertible:
            setattr(module, name, build(child))
        else:
            _convert_recursive(child, mapping, always)


def convert(model: Module, inplace: bool = False) -> Module:
    """Swap calibrated modules for their quantized forms."""
    import lucid_amd.backends as backends
    import lucid_amd.nn as nn
    import lucid_amd.nn.intrinsic as nni
    import lucid_amd.nn.quantized as nnq

    model = model if inplace else copy.deepcopy(model)
    mapping = _quant_mapping()
    if backends.quantized.use_mlx():
        mapping = dict(mapping)
        mapping[nn.Linear] = _mlx_linear_builder(relu=False)
        mapping[nni.LinearReLU] = _mlx_linear_builder(relu=True)
    _convert_recursive(model, mapping, always=(nnq.DeQuantStub, nn.Embedding, nn.EmbeddingBag))
    clear_marks(model)
    model.eval()
    return model


def _dynamic_builders() -> dict:
    import lucid_amd.backends as backends
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized.dynamic as nnqd

    builders = {nn.Linear: nnqd.Linear.from_float, nn.LSTM: nnqd.LSTM.from_float, nn.GRU: nnqd.GRU.from_float,
                nn.LSTMCell: nnqd.LSTMCell.from_float, nn.GRUCell: nnqd.GRUCell.from_float,
                nn.RNNCell: nnqd.RNNCell.from_float}
    if backends.quantized.use_mlx():
        builders[nn.Linear] = _mlx_dynamic_builder()
    return builders


def _replace_dynamic(model: Module, mapping: QConfigMapping, labels: tuple[str, ...],
                     builders: dict, dtype: QDtype) -> Module:
    """Swap every planned site that has a recipe and a dynamic builder for its quantized form,
    parents first (a replaced module's subtree is not visited); returns the (possibly new)
    root.  A module used at several places (a tied layer) is swapped at each of them, by one
    quantized module built at its first place.  Warns when a rule names a leaf module that
    has no dynamic form, or when nothing at all was replaced."""
    sites = plan_sites(model, mapping, every_occurrence=True)
    root = sites[0]
    if root.qconfig is not None and type(model) in builders:
        return builders[type(model)](model, weight_dtype(root.qconfig, dtype))
    replaced: list[str] = []   # paths of replaced modules; their subtrees are skipped
    stays_float: set[type] = set()

    def under_replaced(site: Site) -> bool:
        return any(site.path.startswith(p + ".") for p in replaced)

    built: dict[int, Module] = {}  # id of a float module -> its quantized form
    for site in sites[1:]:
        if under_replaced(site):
            continue
        build = builders.get(type(site.module))
        if site.qconfig is not None and build is not None:
            key = id(site.module)
            if key not in built:
                built[key] = build(site.module, weight_dtype(site.qconfig, dtype))
            setattr(site.parent, site.attr, built[key])
            replaced.append(site.path)
        elif (site.qconfig is not None and next(site.module.children(), None) is None
              and names_a_recipe(mapping, site.module, site.path)):
            stays_float.add(type(site.module))
    if stays_float:
        covered = ", ".join(sorted(t.__name__ for t in builders))
        warnings.warn(f"quantize_dynamic(): {', '.join(sorted(t.__name__ for t in stays_float))} "
                      "has no dynamically quantized form and stays float; dynamic quantization "
                      f"covers {covered}.", stacklevel=3)
    elif not replaced:
        warnings.warn("quantize_dynamic(): no module of a targeted type "
                      f"({', '.join(labels) or 'none'}) found -- the model is returned "
                      "unchanged.", stacklevel=3)
    return model


def quantize_dynamic(model: Module, qconfig_spec=None, dtype: QDtype = qint8,
                     inplace: bool = False) -> Module:
    """Replace ``Linear`` and recurrent layers with dynamically quantized int8 layers."""
    model = model if inplace else copy.deepcopy(model)
    model.eval()
    builders = _dynamic_builders()
    mapping, labels = dynamic_rules(qconfig_spec, dtype, tuple(builders))
    model = _replace_dynamic(model, mapping, labels, builders, dtype)
    clear_marks(model)
    return model
