"""``get_peft_model`` / ``PeftModel`` / ``LoraModel`` for LoRA over this backend's linears
(lucid/peft/_mapping.py:117-170, _peft_model.py:330-1003, tuners/lora/_model.py:127-577).

``get_peft_model(model, config)`` adapts ``model`` in place: every module whose path the
config targets and whose type has a LoRA layer here (``nn.Linear``, ``nnq.Linear``,
``nnqd.Linear``, ``QuantizedLinearMLX``) is replaced by that layer around it, every other
parameter is frozen, and the model comes back wrapped as ``PeftModel`` (``base_model`` the
``LoraModel``, ``base_model.model`` the user's module), so state-dict keys read
``base_model.model.<path>.base_layer...`` and ``...lora_A.<adapter>.weight`` as Lucid's do.
"""

from __future__ import annotations

import contextlib
import copy

from lucid_amd.nn.module import Module
from lucid_amd.peft.lora import Linear, LoraConfig, lora_layer_for


def _lora_layers(model: Module):
    for name, mod in model.named_modules():
        if isinstance(mod, Linear):
            yield name, mod


def _parent_of(model: Module, path: str) -> tuple[Module, str]:
    parent = model
    parts = path.split(".")
    for p in parts[:-1]:
        parent = getattr(parent, p)
    return parent, parts[-1]


class LoraModel(Module):
    """The tuner: holds the adapted model as ``model`` and the configs by adapter name."""

    def __init__(self, model: Module, config: LoraConfig, adapter_name: str = "default") -> None:
        super().__init__()
        self.model = model
        self.peft_config: dict[str, LoraConfig] = {}
        self.active_adapter = adapter_name
        self.add_adapter(adapter_name, config)

    def add_adapter(self, adapter_name: str, config: LoraConfig) -> None:
        if adapter_name in self.peft_config:
            raise ValueError(f"adapter {adapter_name!r} already exists")
        config = copy.deepcopy(config)
        found = False
        inside = [n for n, m in self.model.named_modules() if isinstance(m, Linear)]
        for name, mod in list(self.model.named_modules()):
            if not name or any(name.startswith(p + ".") for p in inside) or not config.matches(name):
                continue
            if isinstance(mod, Linear):  # an adapted layer: one more adapter on it
                mod.update_layer(adapter_name, config)
                found = True
                continue
            parent, attr = _parent_of(self.model, name)
            layer = lora_layer_for(mod, adapter_name, config)
            if layer is None:
                raise ValueError(f"target module {name!r} ({type(mod).__name__}) has no LoRA layer in this "
                                 "backend; supported: Linear, nn.quantized.Linear, "
                                 "nn.quantized.dynamic.Linear, QuantizedLinearMLX")
            setattr(parent, attr, layer)
            found = True
        if not found:
            raise ValueError(f"Target modules {config.target_modules} not found in the base model. "
                             "Please check the target modules and try again.")
        self.peft_config[adapter_name] = config
        for n, p in self.model.named_parameters():
            p.requires_grad = ".lora_A." in f".{n}" or ".lora_B." in f".{n}"

    def set_adapter(self, adapter_name: str) -> None:
        for _, layer in _lora_layers(self.model):
            if adapter_name in layer._specs:
                layer.set_adapter(adapter_name)
        self.active_adapter = adapter_name

    def forward(self, *args, **kwargs):
        return self.model(*args, **kwargs)

    def merge_adapter(self, adapter_names: list[str] | None = None) -> None:
        for _, layer in _lora_layers(self.model):
            layer.merge(adapter_names)

    def unmerge_adapter(self) -> None:
        for _, layer in _lora_layers(self.model):
            layer.unmerge()

    def _replace_layers(self, merge: bool, adapter_names: list[str] | None) -> Module:
        for name, layer in list(_lora_layers(self.model)):
            if merge:
                layer.merge(adapter_names)
            parent, attr = _parent_of(self.model, name)
            setattr(parent, attr, layer.base_layer)
        return self.model

    def merge_and_unload(self, adapter_names: list[str] | None = None) -> Module:
        """Merge the adapters into the base weights and return the plain model."""
        return self._replace_layers(True, adapter_names)

    def unload(self) -> Module:
        """Return the base model with the LoRA layers taken out, unmerged."""
        for _, layer in _lora_layers(self.model):
            layer.unmerge()
        return self._replace_layers(False, None)


class PeftModel(Module):
    """The adapted model (lucid/peft/_peft_model.py:330): forwards to ``base_model``."""

    def __init__(self, model: Module, config: LoraConfig, adapter_name: str = "default") -> None:
        super().__init__()
        self.base_model = LoraModel(model, config, adapter_name)

    @property
    def peft_config(self) -> dict[str, LoraConfig]:
        return self.base_model.peft_config

    @property
    def active_adapter(self) -> str:
        return self.base_model.active_adapter

    def get_base_model(self) -> Module:
        return self.base_model.model

    def forward(self, *args, **kwargs):
        return self.base_model(*args, **kwargs)

    def add_adapter(self, adapter_name: str, config: LoraConfig) -> None:
        self.base_model.add_adapter(adapter_name, config)

    def set_adapter(self, adapter_name: str) -> None:
        self.base_model.set_adapter(adapter_name)

    def merge_adapter(self, adapter_names: list[str] | None = None) -> None:
        self.base_model.merge_adapter(adapter_names)

    def unmerge_adapter(self) -> None:
        self.base_model.unmerge_adapter()

    def merge_and_unload(self, adapter_names: list[str] | None = None) -> Module:
        return self.base_model.merge_and_unload(adapter_names)

    def unload(self) -> Module:
        return self.base_model.unload()

    @contextlib.contextmanager
    def disable_adapter(self):
        """Run the base model alone inside the block."""
        layers = [layer for _, layer in _lora_layers(self.base_model.model)]
        saved = [layer.disable_adapters for layer in layers]
        try:
            for layer in layers:
                layer.disable_adapters = True
            yield
        finally:
            for layer, s in zip(layers, saved):
                layer.disable_adapters = s

    def get_nb_trainable_parameters(self) -> tuple[int, int]:
        trainable = total = 0
        for _, p in self.named_parameters():
            n = p.numel()
            total += n
            if getattr(p, "requires_grad", False):
                trainable += n
        for _, b in self.named_buffers():
            total += b.numel()
        return trainable, total

    def print_trainable_parameters(self) -> None:
        trainable, total = self.get_nb_trainable_parameters()
        print(f"trainable params: {trainable:,d} || all params: {total:,d} || "
              f"trainable%: {100 * trainable / max(total, 1):.4f}")


def get_peft_model(model: Module, peft_config: LoraConfig, adapter_name: str = "default") -> PeftModel:
    """Adapt ``model`` in place with LoRA layers per ``peft_config`` and wrap it."""
    if not isinstance(peft_config, LoraConfig):
        raise TypeError("this backend adapts with LoraConfig only")
    return PeftModel(model, peft_config, adapter_name)
