"""Config-dataclass protocol of the MoE modules.

Mirrors the interface of torchtitan/config/configurable.py:15-113 and
torchtitan/protocols/module.py:23-115 so that ``MoE.Config(...).build()`` and
``init_states`` behave as they do in the reference:

* a component class defines ``Config`` as ``@dataclass(kw_only=True, slots=True)``;
* ``Config.build()`` constructs the owning class with a copy of the config;
* ``Module.init_states`` recurses into children, then runs the per-parameter
  initialisers given by ``Config.param_init`` and ``_init_self_buffers``.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Callable
from dataclasses import dataclass, fields, replace
from typing import ClassVar

import torch
import torch.nn as nn


class Configurable:
    @dataclass(kw_only=True, slots=True)
    class Config:
        _owner: ClassVar[type | None] = None

        def to_dict(self) -> dict:
            def conv(v):
                if hasattr(v, "to_dict"):
                    return v.to_dict()
                if dataclasses.is_dataclass(v):
                    return dataclasses.asdict(v)
                if isinstance(v, (list, tuple)):
                    return type(v)(conv(i) for i in v)
                if isinstance(v, dict):
                    return {k: conv(i) for k, i in v.items()}
                if v is None or isinstance(v, (str, int, float, bool)):
                    return v
                return repr(v)

            return {f.name: conv(getattr(self, f.name)) for f in fields(self)}

        def build(self, **kwargs):
            owner = type(self)._owner
            if owner is None:
                raise NotImplementedError(f"{type(self).__name__} is not attached to a component class")
            if kwargs:
                clash = {f.name for f in fields(self)} & kwargs.keys()
                if clash:
                    raise ValueError(f"build() kwargs {clash} overlap with config fields")
            return owner(config=replace(self), **kwargs)

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        cfg = cls.__dict__.get("Config")
        if cfg is None or not issubclass(cfg, Configurable.Config):
            return
        if "__slots__" not in cfg.__dict__:
            raise TypeError(f"{cls.__name__}.Config must use @dataclass(kw_only=True, slots=True)")
        for f in fields(cfg):
            if f.init and not f.kw_only:
                raise TypeError(f"{cls.__name__}.Config field '{f.name}' must be keyword-only")
        cfg._owner = cls


class Module(nn.Module, Configurable):
    _param_init: dict[str, Callable] | None = None

    @dataclass(kw_only=True, slots=True)
    class Config(Configurable.Config):
        param_init: dict | None = None

        def build(self, **kwargs):
            inst = Configurable.Config.build(self, **kwargs)
            if self.param_init is not None:
                inst._param_init = self.param_init
            return inst

    def init_states(self, *, buffer_device: torch.device | None = None) -> None:
        pending = list(self.children())
        while pending:
            child = pending.pop(0)
            if isinstance(child, Module):
                child.init_states(buffer_device=buffer_device)
            else:
                pending.extend(child.children())
        self._init_self_parameters()
        self._init_self_buffers(buffer_device=buffer_device)

    def _init_self_parameters(self) -> None:
        for name, param in self.named_parameters(recurse=False):
            self._init_param(name, param)

    def _init_param(self, name: str, param: nn.Parameter) -> None:
        if self._param_init is None:
            raise ValueError(f"No param_init found for parameter '{name}' in {type(self).__name__}")
        if name not in self._param_init:
            raise ValueError(
                f"No initializer for parameter '{name}' in {type(self).__name__}; "
                f"available: {list(self._param_init)}"
            )
        self._param_init[name](param)

    def _init_self_buffers(self, *, buffer_device: torch.device | None = None) -> None:
        pass


def called_plainly(*modules: nn.Module) -> bool:
    """True when calling each module would run only its own ``forward``: no
    forward or backward hooks registered on it, and none registered globally.

    A fused path that reads a submodule's parameters instead of calling the
    submodule is taken only then, so that hooks always see the calls they were
    registered for."""
    from torch.nn.modules import module as _m

    if (_m._global_forward_hooks or _m._global_forward_pre_hooks or _m._global_backward_hooks
            or _m._global_backward_pre_hooks):
        return False
    for mod in modules:
        if (mod._forward_hooks or mod._forward_pre_hooks or mod._backward_hooks
                or mod._backward_pre_hooks):
            return False
    return True
