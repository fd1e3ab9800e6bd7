"""Config resolution over a module tree (lucid/quantization/_propagate.py:50-278).

``QConfigResolver`` walks a model depth-first, giving each module its own ``.qconfig``
when it has one, else a rule of the mapping (name or type), else its parent's config.
``prepare`` stamps the result on every module; ``convert`` and ``quantize_dynamic`` strip
it afterwards.  ``normalize_dynamic_spec`` turns ``quantize_dynamic``'s ``qconfig_spec``
(a set of types / names, or a dict to QConfig / QDtype / None) into a mapping.
"""

from __future__ import annotations

from collections.abc import Callable, Collection, Iterator, Mapping
from typing import NamedTuple

from lucid_amd.nn.module import Module
from lucid_amd.quantization._qscheme import QDtype, per_channel_symmetric, quint8
from lucid_amd.quantization.observer import PerChannelMinMaxObserver, PlaceholderObserver
from lucid_amd.quantization.qconfig import QConfig, QConfigMapping

_MISSING = object()


class Resolved(NamedTuple):
    name: str
    module: Module
    path: str
    qconfig: QConfig | None


class QConfigResolver:
    def __init__(self, mapping: QConfigMapping, *, implicit: bool = False) -> None:
        self._mapping = mapping
        self._implicit = implicit

    @classmethod
    def from_argument(cls, qconfig, default: Callable[[], QConfigMapping]) -> "QConfigResolver":
        if qconfig is None:
            return cls(default(), implicit=True)
        if isinstance(qconfig, QConfig):
            return cls(QConfigMapping().set_global(qconfig))
        if isinstance(qconfig, QConfigMapping):
            return cls(qconfig)
        raise TypeError("qconfig must be a QConfig, a QConfigMapping or None; got "
                        f"{type(qconfig).__name__}")

    def is_targeted(self, module: Module, path: str) -> bool:
        return (self._mapping._has_rule(type(module), path)
                and self._mapping.get_qconfig(type(module), path) is not None)

    def resolve(self, module: Module, path: str, inherited: QConfig | None) -> QConfig | None:
        own = getattr(module, "qconfig", _MISSING)
        if own is not _MISSING:
            if own is not None and not isinstance(own, QConfig):
                raise TypeError(f"{path or type(module).__name__}.qconfig must be a QConfig or "
                                f"None; got {type(own).__name__}")
            return own
        if self._mapping._has_rule(type(module), path):
            return self._mapping.get_qconfig(type(module), path)
        return inherited

    @staticmethod
    def stamp(entry: Resolved) -> Resolved:
        entry.module.qconfig = entry.qconfig
        return entry

    @staticmethod
    def strip(model: Module) -> None:
        for module in model.modules():
            if "qconfig" in module.__dict__:
                del module.__dict__["qconfig"]

    def root(self, model: Module) -> Resolved:
        seed = self._mapping._fallback()
        if self._implicit and any("qconfig" in m.__dict__ for m in model.modules()):
            seed = None  # explicit per-module configs opt out of the implicit default
        return Resolved("", model, "", self.resolve(model, "", seed))

    def children(self, module: Module, path: str, qconfig: QConfig | None) -> Iterator[Resolved]:
        for name, child in list(module.named_children()):
            child_path = f"{path}.{name}" if path else name
            yield Resolved(name, child, child_path, self.resolve(child, child_path, qconfig))

    def walk(self, model: Module) -> Iterator[Resolved]:
        seen: set[int] = set()
        stack = [self.root(model)]
        while stack:
            entry = stack.pop()
            if id(entry.module) in seen:
                continue
            seen.add(id(entry.module))
            yield entry
            stack.extend(reversed(list(self.children(entry.module, entry.path, entry.qconfig))))


def dynamic_qconfig(dtype: QDtype) -> QConfig:
    return QConfig(
        activation=PlaceholderObserver.with_args(qdtype=quint8),
        weight=PerChannelMinMaxObserver.with_args(ch_axis=0, qscheme=per_channel_symmetric,
                                                  qdtype=dtype),
    )


def weight_dtype(qconfig: QConfig, fallback: QDtype) -> QDtype:
    found = getattr(qconfig.weight(), "qdtype", None)
    return found if isinstance(found, QDtype) else fallback


class DynamicSpec(NamedTuple):
    mapping: QConfigMapping
    targets: tuple[str, ...]


def _spec_value(key: object, value: object) -> QConfig | None:
    if value is None or isinstance(value, QConfig):
        return value
    if isinstance(value, QDtype):
        return dynamic_qconfig(value)
    raise TypeError(f"qconfig_spec[{key!r}] must be a QConfig, a QDtype or None; got "
                    f"{type(value).__name__}")


def normalize_dynamic_spec(spec: object, dtype: QDtype,
                           default_types: Collection[type]) -> DynamicSpec:
    default = dynamic_qconfig(dtype)
    if spec is None:
        entries = dict.fromkeys(default_types, default)
    elif isinstance(spec, Mapping):
        entries = {key: _spec_value(key, value) for key, value in spec.items()}
    elif isinstance(spec, Collection) and not isinstance(spec, (str, type)):
        entries = dict.fromkeys(spec, default)
    else:
        raise TypeError("qconfig_spec must be a set of module types / names or a dict mapping "
                        f"them to a QConfig, a QDtype or None; got {type(spec).__name__}")
    mapping = QConfigMapping()
    targets: list[str] = []
    for key, qconfig in entries.items():
        if isinstance(key, str):
            mapping.set_module_name(key, qconfig)
            label = key
        elif isinstance(key, type) and issubclass(key, Module):
            mapping.set_object_type(key, qconfig)
            label = key.__name__
        else:
            raise TypeError(f"qconfig_spec keys must be nn.Module subclasses or module names; "
                            f"got {key!r}")
        if qconfig is not None:
            targets.append(label)
    return DynamicSpec(mapping, tuple(sorted(targets)))
