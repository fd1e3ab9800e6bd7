"""``nn.Module``: the parts of Lucid's module system the quantized path relies on.

Parameters, buffers and sub-modules in insertion order, ``state_dict`` /
``load_state_dict`` (with the ``_load_from_state_dict`` hook observers override),
forward hooks (``prepare`` attaches observers through them), ``train``/``eval``,
``to(device)`` and the ``named_*`` walkers.  Behaviour follows
lucid/nn/module.py (buffer registration keeps a re-registered name in place,
module.py:904-921).
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any, Callable, Iterator

from lucid_amd._tensor import Tensor, normalize_device


class Parameter(Tensor):
    """A tensor registered as a module parameter."""

    __slots__ = ()

    def __new__(cls, data: Tensor | None = None, requires_grad: bool = True) -> "Parameter":
        obj = Tensor.__new__(cls)
        Tensor.__init__(obj)
        if data is not None:
            obj._host = data._host
            obj._buf = data._buf
            obj._offset = data._offset
            obj._shape = data._shape
            obj._dtype = data._dtype
            obj._device = data._device
            obj._qsrc = data._qsrc
        obj.requires_grad = requires_grad
        return obj

    def __init__(self, data: Tensor | None = None, requires_grad: bool = True) -> None:
        pass


class _RemovableHandle:
    def __init__(self, hooks: dict, key: int) -> None:
        self._hooks = hooks
        self._key = key

    def remove(self) -> None:
        self._hooks.pop(self._key, None)


class Module:
    _next_hook_id = 0

    def __init__(self) -> None:
        object.__setattr__(self, "_parameters", OrderedDict())
        object.__setattr__(self, "_buffers", OrderedDict())
        object.__setattr__(self, "_non_persistent", set())
        object.__setattr__(self, "_modules", OrderedDict())
        object.__setattr__(self, "_forward_hooks", OrderedDict())
        object.__setattr__(self, "_forward_pre_hooks", OrderedDict())
        object.__setattr__(self, "training", True)

    # ---------------------------------------------------------- registration
    def register_buffer(self, name: str, tensor: Tensor | None, persistent: bool = True) -> None:
        if "_buffers" not in self.__dict__:
            raise AttributeError("Module.__init__() was not called")
        if tensor is not None and not isinstance(tensor, Tensor):
            raise TypeError(f"buffer {name!r} must be a Tensor or None")
        for store in (self._parameters, self._modules):
            store.pop(name, None)
        if name in self.__dict__:
            object.__delattr__(self, name)
        self._buffers[name] = tensor  # an existing key keeps its position
        if persistent:
            self._non_persistent.discard(name)
        else:
            self._non_persistent.add(name)

    def register_parameter(self, name: str, param: Parameter | None) -> None:
        if param is not None and not isinstance(param, Parameter):
            param = Parameter(param)
        for store in (self._buffers, self._modules):
            store.pop(name, None)
        self._parameters[name] = param

    def add_module(self, name: str, module: "Module | None") -> None:
        for store in (self._parameters, self._buffers):
            store.pop(name, None)
        self._modules[name] = module

    def __setattr__(self, name: str, value: Any) -> None:
        d = self.__dict__
        if "_parameters" not in d:
            object.__setattr__(self, name, value)
            return
        if isinstance(value, Parameter):
            d.pop(name, None)
            self.register_parameter(name, value)
        elif isinstance(value, Module):
            d.pop(name, None)
            self.add_module(name, value)
        elif name in self._parameters:
            if value is not None and not isinstance(value, Tensor):
                raise TypeError(f"cannot assign {type(value).__name__} to parameter {name!r}")
            self._parameters[name] = None if value is None else Parameter(value)
        elif name in self._buffers:
            if value is not None and not isinstance(value, Tensor):
                raise TypeError(f"cannot assign {type(value).__name__} to buffer {name!r}")
            self._buffers[name] = value
        elif name in self._modules and value is None:
            self._modules[name] = None
        else:
            object.__setattr__(self, name, value)

    def __getattr__(self, name: str) -> Any:
        d = self.__dict__
        for store in ("_parameters", "_buffers", "_modules"):
            s = d.get(store)
            if s is not None and name in s:
                return s[name]
        raise AttributeError(f"{type(self).__name__!r} object has no attribute {name!r}")

    def __delattr__(self, name: str) -> None:
        for store in (self._parameters, self._buffers, self._modules):
            if name in store:
                del store[name]
                return
        object.__delattr__(self, name)

    # --------------------------------------------------------------- walkers
    def named_children(self) -> Iterator[tuple[str, "Module"]]:
        for name, m in self._modules.items():
            if m is not None:
                yield name, m

    def children(self) -> Iterator["Module"]:
        for _, m in self.named_children():
            yield m

    def named_modules(self, prefix: str = "", memo: set | None = None) -> Iterator[tuple[str, "Module"]]:
        memo = set() if memo is None else memo
        if id(self) in memo:
            return
        memo.add(id(self))
        yield prefix, self
        for name, m in self.named_children():
            yield from m.named_modules(f"{prefix}.{name}" if prefix else name, memo)

    def modules(self) -> Iterator["Module"]:
        for _, m in self.named_modules():
            yield m

    def named_parameters(self, prefix: str = "", recurse: bool = True) -> Iterator[tuple[str, Parameter]]:
        mods = self.named_modules(prefix) if recurse else [(prefix, self)]
        for mp, m in mods:
            for n, p in m._parameters.items():
                if p is not None:
                    yield (f"{mp}.{n}" if mp else n), p

    def parameters(self, recurse: bool = True) -> Iterator[Parameter]:
        for _, p in self.named_parameters(recurse=recurse):
            yield p

    def named_buffers(self, prefix: str = "", recurse: bool = True) -> Iterator[tuple[str, Tensor]]:
        mods = self.named_modules(prefix) if recurse else [(prefix, self)]
        for mp, m in mods:
            for n, b in m._buffers.items():
                if b is not None:
                    yield (f"{mp}.{n}" if mp else n), b

    def buffers(self, recurse: bool = True) -> Iterator[Tensor]:
        for _, b in self.named_buffers(recurse=recurse):
            yield b

    def apply(self, fn: Callable[["Module"], None]) -> "Module":
        for m in self.children():
            m.apply(fn)
        fn(self)
        return self

    # ------------------------------------------------------------ state dict
    def state_dict(self, prefix: str = "") -> "OrderedDict[str, Tensor]":
        out: OrderedDict[str, Tensor] = OrderedDict()
        self._save_to_state_dict(out, prefix)
        for name, m in self.named_children():
            out.update(m.state_dict(prefix=f"{prefix}{name}."))
        return out

    def _save_to_state_dict(self, dest: dict, prefix: str) -> None:
        for n, p in self._parameters.items():
            if p is not None:
                dest[prefix + n] = p
        for n, b in self._buffers.items():
            if b is not None and n not in self._non_persistent:
                dest[prefix + n] = b

    def _load_from_state_dict(self, state_dict: dict, prefix: str, local_metadata: dict,
                              strict: bool, missing_keys: list, unexpected_keys: list,
                              error_msgs: list) -> None:
        local = {**{n: p for n, p in self._parameters.items() if p is not None},
                 **{n: b for n, b in self._buffers.items()
                    if b is not None and n not in self._non_persistent}}
        for name, cur in local.items():
            key = prefix + name
            if key not in state_dict:
                missing_keys.append(key)
                continue
            src = state_dict[key]
            if tuple(src.shape) != tuple(cur.shape):
                error_msgs.append(f"size mismatch for {key}: copying {tuple(src.shape)} into "
                                  f"{tuple(cur.shape)}")
                continue
            if src.dtype != cur.dtype:
                error_msgs.append(f"dtype mismatch for {key}: {src.dtype} vs {cur.dtype}")
                continue
            cur.copy_(src)
        if strict:
            for key in state_dict:
                if key.startswith(prefix):
                    rest = key[len(prefix):]
                    head = rest.split(".", 1)[0]
                    if "." not in rest and head not in local:
                        unexpected_keys.append(key)
                    elif "." in rest and head not in self._modules:
                        unexpected_keys.append(key)

    def load_state_dict(self, state_dict: dict, strict: bool = True) -> tuple[list, list]:
        missing: list = []
        unexpected: list = []
        errors: list = []

        def load(m: Module, prefix: str) -> None:
            m._load_from_state_dict(state_dict, prefix, {}, strict, missing, unexpected, errors)
            for name, child in m.named_children():
                load(child, f"{prefix}{name}.")

        load(self, "")
        if strict and (missing or unexpected):
            errors.insert(0, f"missing keys {missing}, unexpected keys {unexpected}")
        if errors:
            raise RuntimeError("Error(s) in loading state_dict:\n  " + "\n  ".join(errors))
        return missing, unexpected

    # ----------------------------------------------------------------- modes
    def train(self, mode: bool = True) -> "Module":
        object.__setattr__(self, "training", mode)
        for m in self.children():
            m.train(mode)
        return self

    def eval(self) -> "Module":
        return self.train(False)

    def to(self, device: Any) -> "Module":
        dev = normalize_device(device)
        for m in self.modules():
            for n, p in list(m._parameters.items()):
                if p is not None and p.device != dev:
                    m._parameters[n] = Parameter(p.to(dev), p.requires_grad)
            for n, b in list(m._buffers.items()):
                if b is not None and b.device != dev:
                    m._buffers[n] = b.to(dev)
        return self

    def cpu(self) -> "Module":
        return self.to("cpu")

    def gpu(self) -> "Module":
        return self.to("gpu")

    # ------------------------------------------------------------------ hooks
    def register_forward_hook(self, hook: Callable) -> _RemovableHandle:
        Module._next_hook_id += 1
        self._forward_hooks[Module._next_hook_id] = hook
        return _RemovableHandle(self._forward_hooks, Module._next_hook_id)

    def register_forward_pre_hook(self, hook: Callable) -> _RemovableHandle:
        Module._next_hook_id += 1
        self._forward_pre_hooks[Module._next_hook_id] = hook
        return _RemovableHandle(self._forward_pre_hooks, Module._next_hook_id)

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        raise NotImplementedError(f"{type(self).__name__}.forward")

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        if self._forward_pre_hooks:
            for hook in list(self._forward_pre_hooks.values()):
                r = hook(self, args)
                if r is not None:
                    args = r if isinstance(r, tuple) else (r,)
        out = self.forward(*args, **kwargs)
        if self._forward_hooks:
            for hook in list(self._forward_hooks.values()):
                r = hook(self, args, out)
                if r is not None:
                    out = r
        return out

    # ------------------------------------------------------------------- repr
    def extra_repr(self) -> str:
        return ""

    def __repr__(self) -> str:
        lines = [f"{type(self).__name__}({self.extra_repr()}"]
        kids = list(self.named_children())
        if not kids:
            return lines[0] + ")"
        for name, m in kids:
            sub = repr(m).replace("\n", "\n  ")
            lines.append(f"  ({name}): {sub}")
        return "\n".join(lines) + "\n)"
