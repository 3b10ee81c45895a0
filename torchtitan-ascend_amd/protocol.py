"""TorchTitan protocol the converters plug into.

When `torchtitan` is importable its own classes are used.  Otherwise (as on
every machine this build runs on) a minimal stand-in with the same names and
semantics is defined here, so converters, configs and modules work without
it:

  Module / Module.Config.build()     torchtitan.protocols.module.Module
  ModelConfigConverter(.Config)      torchtitan.protocols.model.ModelConfigConverter
  ModelConfig.traverse(cls)          yields (fqn, cfg, parent, attr)
  GroupedExperts.Config              torchtitan.models.common.moe.GroupedExperts
  AllToAllTokenDispatcher.Config     torchtitan.models.common.token_dispatcher

The stand-in upstream modules (GroupedExperts, the upstream dispatchers)
carry only their configs: their forward raises, because the upstream
implementation is not part of this build.  Converted modules never call them.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Any, Iterator

from torch import nn

try:  # pragma: no cover - torchtitan is absent on the build and GPU machines
    from torchtitan.models.common.moe import GroupedExperts  # type: ignore
    from torchtitan.models.common.token_dispatcher import AllToAllTokenDispatcher  # type: ignore
    from torchtitan.protocols.model import ModelConfig, ModelConfigConverter  # type: ignore
    from torchtitan.protocols.module import Module  # type: ignore

    HAVE_TORCHTITAN = True
    LocalTokenDispatcher = AllToAllTokenDispatcher
except ImportError:
    HAVE_TORCHTITAN = False

    class Module(nn.Module):
        """nn.Module whose nested dataclass `Config` builds it."""

        @dataclass(kw_only=True, slots=True)
        class Config:
            def build(self, **kwargs):
                owner = getattr(type(self), "_owner", None)
                if owner is None:
                    raise TypeError(f"{type(self).__qualname__} is not attached to a Module")
                return owner(self, **kwargs)

        def __init_subclass__(cls, **kwargs):
            super().__init_subclass__(**kwargs)
            cfg = cls.__dict__.get("Config")
            if cfg is not None:
                cfg._owner = cls

    class ModelConfigConverter:
        """Rewrites configs inside a model config before the model is built."""

        @dataclass(kw_only=True, slots=True)
        class Config:
            def build(self, **kwargs):
                owner = getattr(type(self), "_owner", None)
                if owner is None:
                    raise TypeError(f"{type(self).__qualname__} is not attached to a converter")
                return owner(self, **kwargs)

        def __init_subclass__(cls, **kwargs):
            super().__init_subclass__(**kwargs)
            cfg = cls.__dict__.get("Config")
            if cfg is not None:
                cfg._owner = cls

        def __init__(self, config: "ModelConfigConverter.Config"):
            self.config = config

        def convert(self, model_config) -> None:
            raise NotImplementedError

    def _children(obj: Any) -> Iterator[tuple[str, Any]]:
        if dataclasses.is_dataclass(obj) and not isinstance(obj, type):
            for f in dataclasses.fields(obj):
                yield f.name, getattr(obj, f.name, None)
        if hasattr(obj, "__dict__") and not isinstance(obj, type):
            seen = {f.name for f in dataclasses.fields(obj)} if dataclasses.is_dataclass(obj) else set()
            for k, v in vars(obj).items():
                if k not in seen and not k.startswith("_"):
                    yield k, v

    class ModelConfig:
        """Container of module configs; `traverse` finds configs by type."""

        def traverse(self, cls: type) -> Iterator[tuple[str, Any, Any, Any]]:
            """Yield (fqn, cfg, parent, attr) for every instance of `cls` below
            this config; parent[attr] (list) or getattr(parent, attr) is cfg.
            Matches are collected first, so callers may replace them."""
            found: list[tuple[str, Any, Any, Any]] = []
            seen: set[int] = set()

            def walk(obj, fqn):
                if id(obj) in seen:
                    return
                seen.add(id(obj))
                if isinstance(obj, (list, tuple)):
                    items = list(enumerate(obj))
                    for i, v in items:
                        name = f"{fqn}.{i}" if fqn else str(i)
                        if isinstance(v, cls):
                            found.append((name, v, obj, i))
                        if _is_node(v):
                            walk(v, name)
                    return
                for k, v in _children(obj):
                    name = f"{fqn}.{k}" if fqn else k
                    if isinstance(v, cls):
                        found.append((name, v, obj, k))
                    if _is_node(v):
                        walk(v, name)

            walk(self, "")
            yield from found

    def _is_node(v: Any) -> bool:
        return isinstance(v, (list, tuple)) or (
            not isinstance(v, (str, bytes, int, float, bool, type(None))) and
            (dataclasses.is_dataclass(v) or isinstance(v, ModelConfig))
        )

    class LocalTokenDispatcher(Module):
        """Stand-in for upstream's local (single-rank) token dispatcher config."""

        @dataclass(kw_only=True, slots=True)
        class Config(Module.Config):
            num_experts: int
            top_k: int
            score_before_experts: bool = True

        def __init__(self, config: "LocalTokenDispatcher.Config"):
            super().__init__()
            self.num_experts = config.num_experts
            self.top_k = config.top_k
            self.score_before_experts = config.score_before_experts

        def dispatch(self, x, top_scores, selected_experts_indices):
            raise NotImplementedError(
                "the upstream TorchTitan dispatcher is not installed; convert it with "
                "HipTokenDispatcherConverter"
            )

        def combine(self, routed_output, metadata, x):
            raise NotImplementedError(
                "the upstream TorchTitan dispatcher is not installed; convert it with "
                "HipTokenDispatcherConverter"
            )

    class AllToAllTokenDispatcher(LocalTokenDispatcher):
        """Stand-in for upstream AllToAllTokenDispatcher (expert-parallel)."""

        @dataclass(kw_only=True, slots=True)
        class Config(LocalTokenDispatcher.Config):
            pass

    class GroupedExperts(Module):
        """Stand-in for upstream GroupedExperts (w1/w3 [E,H,D], w2 [E,D,H])."""

        @dataclass(kw_only=True, slots=True)
        class Config(Module.Config):
            dim: int
            hidden_dim: int
            num_experts: int
            token_dispatcher: LocalTokenDispatcher.Config
            use_grouped_mm: bool = True

        def __init__(self, config: "GroupedExperts.Config"):
            super().__init__()
            self.config = config

        def forward(self, *args, **kwargs):
            raise NotImplementedError(
                "the upstream TorchTitan GroupedExperts is not installed; convert it with "
                "HipGroupedExpertsConverter"
            )


__all__ = [
    "HAVE_TORCHTITAN",
    "Module",
    "ModelConfig",
    "ModelConfigConverter",
    "GroupedExperts",
    "LocalTokenDispatcher",
    "AllToAllTokenDispatcher",
]
