"""``QConfig`` / ``QConfigMapping`` and the stock configs (lucid/quantization/qconfig.py:30-512).

A ``QConfig`` is a pair of observer factories (activation, weight).  ``QConfigMapping``
resolves a module's config by precedence: module name > module type > global
(qconfig.py:430-470).  ``get_default_qconfig`` is Lucid's static PTQ default: a
``HistogramObserver`` for activations and a per-channel symmetric ``qint8`` weight observer.
"""

from __future__ import annotations

from typing import Callable, NamedTuple

from lucid_amd.quantization._qscheme import (per_channel_symmetric, per_tensor_affine, qint8,
                                             quint8)
from lucid_amd.quantization.observer import (HistogramObserver, MinMaxObserver,
                                             PerChannelMinMaxObserver)

_Factory = Callable[..., object]


class QConfig(NamedTuple):
    activation: _Factory
    weight: _Factory


def get_default_qconfig() -> QConfig:
    return QConfig(
        activation=HistogramObserver.with_args(qscheme=per_tensor_affine, qdtype=quint8),
        weight=PerChannelMinMaxObserver.with_args(ch_axis=0, qscheme=per_channel_symmetric,
                                                  qdtype=qint8),
    )


def get_minmax_qconfig() -> QConfig:
    """Static PTQ with a ``MinMaxObserver`` on activations (the pinned-observer variant
    of the default)."""
    return QConfig(
        activation=MinMaxObserver.with_args(qscheme=per_tensor_affine, qdtype=quint8),
        weight=PerChannelMinMaxObserver.with_args(ch_axis=0, qscheme=per_channel_symmetric,
                                                  qdtype=qint8),
    )


class QConfigMapping:
    """Per-module config resolution: module name > module type > global."""

    def __init__(self) -> None:
        self._global: QConfig | None = None
        self._object_type: dict[type, QConfig | None] = {}
        self._module_name: dict[str, QConfig | None] = {}

    def set_global(self, qconfig: QConfig | None) -> "QConfigMapping":
        self._global = qconfig
        return self

    def set_object_type(self, module_type: type, qconfig: QConfig | None) -> "QConfigMapping":
        self._object_type[module_type] = qconfig
        return self

    def set_module_name(self, name: str, qconfig: QConfig | None) -> "QConfigMapping":
        self._module_name[name] = qconfig
        return self

    def get_qconfig(self, module_type: type, module_name: str) -> QConfig | None:
        ruled, qconfig = self.rule_for(module_type, module_name)
        return qconfig if ruled else self._global

    def rule_for(self, module_type: type, module_name: str) -> tuple[bool, QConfig | None]:
        """(whether a name or type rule covers the module, its recipe): name before type."""
        for table, key in ((self._module_name, module_name), (self._object_type, module_type)):
            if key in table:
                return True, table[key]
        return False, None

    def global_qconfig(self) -> QConfig | None:
        return self._global


def get_default_qconfig_mapping() -> QConfigMapping:
    return QConfigMapping().set_global(get_default_qconfig())
