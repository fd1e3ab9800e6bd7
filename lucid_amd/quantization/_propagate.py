"""Which ``QConfig`` applies to each module of a model.

Lucid resolves a module's recipe in three tiers (lucid/quantization/_propagate.py:50-278,
the behaviour this file keeps): the module's own ``.qconfig`` attribute if it has one (a
``QConfig``, or ``None`` to exclude it), else a per-name or per-type rule of the
``QConfigMapping`` (name before type), else whatever its parent resolved to.  The root
inherits the mapping's global recipe -- except when the caller passed no config at all
(the entry point's stock default) and the model already carries ``.qconfig`` attributes:
then the user has configured modules, and the stock recipe does not cover the rest.

Here that is one pure function, :func:`plan_sites`, which returns every module once in
parent-before-child order as a :class:`Site` (where it hangs in its parent, its dotted
path and its recipe).  ``prepare`` marks and observes modules from the plan;
``quantize_dynamic`` replaces modules from it.  Nothing is written during planning.
"""

from __future__ import annotations

from collections.abc import Callable, Collection, Mapping
from dataclasses import dataclass

from lucid_amd.nn.module import Module
from lucid_amd.quantization._qscheme import QDtype, per_channel_symmetric, quint8
from lucid_amd.quantization.observer import PerChannelMinMaxObserver, PlaceholderObserver
from lucid_amd.quantization.qconfig import QConfig, QConfigMapping

MARK = "qconfig"  # the per-module attribute the tiers read and prepare writes


@dataclass(frozen=True)
class Site:
    """One module of a model and the recipe it resolved to (``None``: stays float)."""

    parent: Module | None  # None for the root
    attr: str              # attribute name in the parent ("" for the root)
    module: Module
    path: str              # dotted path from the root ("" for the root)
    qconfig: QConfig | None


def as_mapping(qconfig: object, default: Callable[[], QConfigMapping]) -> tuple[QConfigMapping, bool]:
    """The mapping an entry point's ``qconfig`` argument denotes, and whether it is the stock
    default (``qconfig is None``).  A bare ``QConfig`` is the global tier."""
    if qconfig is None:
        return default(), True
    if isinstance(qconfig, QConfigMapping):
        return qconfig, False
    if isinstance(qconfig, QConfig):
        return QConfigMapping().set_global(qconfig), False
    raise TypeError("qconfig must be a QConfig, a QConfigMapping or None; got "
                    f"{type(qconfig).__name__}")


_ABSENT = object()


def _own(module: Module, path: str) -> tuple[bool, QConfig | None]:
    """(has its own recipe, that recipe) from the module's ``.qconfig`` attribute."""
    own = getattr(module, MARK, _ABSENT)
    if own is _ABSENT:
        return False, None
    if own is not None and not isinstance(own, QConfig):
        raise TypeError(f"{path or type(module).__name__}.qconfig must be a QConfig or None; got "
                        f"{type(own).__name__}")
    return True, own


def recipe_for(mapping: QConfigMapping, module: Module, path: str,
               inherited: QConfig | None) -> QConfig | None:
    """The effective recipe of one module given its parent's."""
    has_own, own = _own(module, path)
    if has_own:
        return own
    ruled, qconfig = mapping.rule_for(type(module), path)
    return qconfig if ruled else inherited


def names_a_recipe(mapping: QConfigMapping, module: Module, path: str) -> bool:
    """Whether a per-name / per-type rule names this module with a (non-None) recipe."""
    ruled, qconfig = mapping.rule_for(type(module), path)
    return ruled and qconfig is not None


def plan_sites(model: Module, mapping: QConfigMapping, *, stock_default: bool = False,
               every_occurrence: bool = False) -> list[Site]:
    """Every module of ``model``, parents before children and children in registration
    order, each with its resolved recipe.  A module reachable along two paths is taken at its
    first only, unless ``every_occurrence``: then each (parent, attribute) slot is a site of
    its own (a tied layer is swapped in every place it is used; only a module that contains
    itself is cut off)."""
    seed = mapping.global_qconfig()
    if stock_default and any(hasattr(m, MARK) for m in model.modules()):
        seed = None  # the user configured modules: the stock default does not fill in
    sites: list[Site] = []
    visited: set[int] = set()

    def visit(parent: Module | None, attr: str, module: Module, path: str,
              inherited: QConfig | None) -> None:
        if id(module) in visited:
            return
        visited.add(id(module))
        qconfig = recipe_for(mapping, module, path, inherited)
        sites.append(Site(parent, attr, module, path, qconfig))
        for name, child in list(module.named_children()):
            visit(module, name, child, f"{path}.{name}" if path else name, qconfig)
        if every_occurrence:
            visited.discard(id(module))  # ancestors only: siblings may hold it again

    visit(None, "", model, "", seed)
    return sites


def mark(sites: list[Site]) -> None:
    """Write each site's recipe onto its module (``None`` marks an exclusion)."""
    for site in sites:
        setattr(site.module, MARK, site.qconfig)


def clear_marks(model: Module) -> None:
    """Remove every module's ``.qconfig`` attribute: after conversion the marks mean nothing,
    and a later ``prepare`` would read leftovers as the user's own per-module choices."""
    for module in model.modules():
        module.__dict__.pop(MARK, None)


# ------------------------------------------------------------------ quantize_dynamic specs


def dynamic_qconfig(dtype: QDtype) -> QConfig:
    """quantize_dynamic's recipe for weight dtype ``dtype``: a placeholder activation observer
    (activations are quantized at run time) and a per-output-channel symmetric weight
    observer on ``dtype``'s grid."""
    return QConfig(
        activation=PlaceholderObserver.with_args(qdtype=quint8),
        weight=PerChannelMinMaxObserver.with_args(ch_axis=0, qscheme=per_channel_symmetric,
                                                  qdtype=dtype),
    )


def weight_dtype(qconfig: QConfig, fallback: QDtype) -> QDtype:
    """The weight grid a recipe asks for (its weight observer's ``qdtype``), else ``fallback``."""
    qdtype = getattr(qconfig.weight(), "qdtype", None)
    return qdtype if isinstance(qdtype, QDtype) else fallback


def _recipe_of_value(key: object, value: object) -> QConfig | None:
    if isinstance(value, QDtype):
        return dynamic_qconfig(value)
    if value is None or isinstance(value, QConfig):
        return value
    raise TypeError(f"qconfig_spec[{key!r}] must be a QConfig, a QDtype or None; got "
                    f"{type(value).__name__}")


def dynamic_rules(spec: object, dtype: QDtype,
                  default_types: Collection[type]) -> tuple[QConfigMapping, tuple[str, ...]]:
    """``quantize_dynamic``'s ``qconfig_spec`` as a mapping, plus the sorted labels of what it
    asks to quantize (for messages).  ``None`` targets ``default_types``; a collection of
    module types and / or dotted names targets each with ``dtype``'s recipe; a dict pairs
    each with a ``QConfig``, a ``QDtype`` or ``None`` (leave float)."""
    if spec is None:
        pairs = [(t, dynamic_qconfig(dtype)) for t in default_types]
    elif isinstance(spec, Mapping):
        pairs = [(key, _recipe_of_value(key, value)) for key, value in spec.items()]
    elif isinstance(spec, Collection) and not isinstance(spec, (str, type)):
        recipe = dynamic_qconfig(dtype)
        pairs = [(key, recipe) for key in spec]
    else:
        raise TypeError("qconfig_spec must be a set of module types / names or a dict mapping "
                        f"them to a QConfig, a QDtype or None; got {type(spec).__name__}")
    mapping = QConfigMapping()
    labels: list[str] = []
    for key, recipe in pairs:
        if isinstance(key, type) and issubclass(key, Module):
            mapping.set_object_type(key, recipe)
            label = key.__name__
        elif isinstance(key, str):
            mapping.set_module_name(key, recipe)
            label = key
        else:
            raise TypeError(f"qconfig_spec keys must be nn.Module subclasses or module names; "
                            f"got {key!r}")
        if recipe is not None:
            labels.append(label)
    return mapping, tuple(sorted(labels))
