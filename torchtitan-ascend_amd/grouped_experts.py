"""HipGroupedExperts and its converter: the expert FFN of the MoE path.

Mirrors torchtitanturbo/models/common/npu_gmm.py:
  * HipGroupedExperts            <- NpuGroupedExperts (:43-115): fused
    w13 [E, 2H, D] (rows 0..H-1 gate, H..2H-1 up) and w2 [E, D, H]
  * run_experts_grouped_mm       <- _run_experts_grouped_mm (:21-40)
  * HipGroupedExpertsConverter   <- NpuGroupedExpertsConverter (:118-152)

The grouped GEMMs, the SwiGLU (+ clamp) epilogue and the fused
scale + un-permute epilogue are hand-written gfx950 kernels
(libttamd_moe.so).  Single GPU only: expert tensor parallelism (the
reference's all_reduce at :93-96) is not part of this build.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

from .functional import moe_experts_forward, run_experts_grouped_mm
from .protocol import GroupedExperts, Module, ModelConfigConverter
from .state_dict import upstream_to_fused
from .token_dispatcher import HipTokenDispatcher


def _local(p: torch.Tensor) -> tuple[torch.Tensor, int]:
    """DTensor -> (local shard, expert-TP degree): the number of shards the
    hidden dim (dim 2 of w2) is split into, 1 when it is not split
    (npu_gmm.py:74-83 detects the same Shard(2) placement)."""
    try:
        from torch.distributed.tensor import DTensor
        from torch.distributed.tensor.placement_types import Shard
    except ImportError:  # pragma: no cover
        return p, 1
    if isinstance(p, DTensor):
        tp = 1
        for mesh_dim, pl in enumerate(p.placements):
            if isinstance(pl, Shard) and pl.dim == 2:
                tp *= p.device_mesh.size(mesh_dim)
        return p.to_local(), tp
    return p, 1


def _load_upstream_w1_w3(state_dict, prefix, *args, **kwargs):
    """load_state_dict pre-hook: {prefix}w1 + {prefix}w3 -> {prefix}w13."""
    if prefix + "w1" in state_dict and prefix + "w13" not in state_dict:
        fused = upstream_to_fused({k: state_dict[k] for k in (prefix + "w1", prefix + "w3")}, prefix)
        del state_dict[prefix + "w1"], state_dict[prefix + "w3"]
        state_dict[prefix + "w13"] = fused[prefix + "w13"]


class HipGroupedExperts(Module):
    """Grouped-expert SwiGLU FFN with a fused w13 parameter, on MI355X kernels."""

    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        dim: int
        hidden_dim: int
        num_experts: int
        token_dispatcher: Any
        swiglu_limit: float | None = None

    def __init__(self, config: "HipGroupedExperts.Config"):
        super().__init__()
        self.num_experts = config.num_experts
        self.swiglu_limit = config.swiglu_limit
        E, D, H = config.num_experts, config.dim, config.hidden_dim
        self.w13 = nn.Parameter(torch.empty(E, 2 * H, D))
        self.w2 = nn.Parameter(torch.empty(E, D, H))
        self.token_dispatcher = config.token_dispatcher.build()
        # checkpoints of upstream GroupedExperts (w1 / w3 [E, H, D]) load as w13
        self._register_load_state_dict_pre_hook(_load_upstream_w1_w3)

    def _weights(self):
        w2, tp2 = _local(self.w2)
        w13, _ = _local(self.w13)
        if tp2 > 1:
            # npu_gmm.py:93-96 all-reduces the partial outputs over the TP
            # group; a mesh of one rank holds the whole hidden dim and runs
            # as is
            raise NotImplementedError(
                f"expert tensor parallelism of degree {tp2} (w2 sharded on dim 2) needs an all-reduce "
                "across the TP group; this build runs the experts of one GPU")
        return w13, w2

    def _experts_forward(self, x, num_tokens_per_expert):
        w13, w2 = self._weights()
        return run_experts_grouped_mm(w13, w2, x, num_tokens_per_expert, self.swiglu_limit)

    def forward(self, x, top_scores, selected_experts_indices):
        bs, slen, dim = x.shape
        top_k = top_scores.size(-1)
        x = x.view(bs * slen, dim)
        top_scores = top_scores.view(bs * slen, top_k)
        selected_experts_indices = selected_experts_indices.view(bs * slen, top_k)
        disp = self.token_dispatcher
        if isinstance(disp, HipTokenDispatcher) and disp.is_local:
            w13, w2 = self._weights()
            return moe_experts_forward(
                x, top_scores, selected_experts_indices, w13, w2, self.num_experts,
                disp.score_before_experts, self.swiglu_limit,
            )
        routed_input, num_tokens_local, metadata = disp.dispatch(x, top_scores, selected_experts_indices)
        routed_output = self._experts_forward(routed_input, num_tokens_local)
        return disp.combine(routed_output, metadata, x)

    def _init_self_parameters(self):
        for name, param in self.named_parameters(recurse=False):
            if name in ("w13", "w2"):
                nn.init.normal_(param, mean=0.0, std=0.02)

    def init_weights(self, *args, **kwargs):
        self._init_self_parameters()


class HipGroupedExpertsConverter(ModelConfigConverter):
    """Replace GroupedExperts configs with HipGroupedExperts configs."""

    @dataclass(kw_only=True, slots=True)
    class Config(ModelConfigConverter.Config):
        swiglu_limit: float | None = None

    def __init__(self, config: "HipGroupedExpertsConverter.Config"):
        self.config = config
        self.swiglu_limit = config.swiglu_limit

    def convert(self, model_config) -> None:
        count = 0
        for _fqn, cfg, parent, attr in model_config.traverse(GroupedExperts.Config):
            new_config = HipGroupedExperts.Config(
                dim=cfg.dim,
                hidden_dim=cfg.hidden_dim,
                num_experts=cfg.num_experts,
                token_dispatcher=cfg.token_dispatcher,
                swiglu_limit=self.swiglu_limit,
            )
            for extra in ("param_init", "sharding_config"):
                if hasattr(cfg, extra):
                    try:
                        setattr(new_config, extra, getattr(cfg, extra))
                    except AttributeError:
                        pass  # slots config without that field
            if isinstance(parent, list):
                parent[attr] = new_config
            else:
                setattr(parent, attr, new_config)
            count += 1
        self.num_converted = count


__all__ = [
    "HipGroupedExperts",
    "HipGroupedExpertsConverter",
    "run_experts_grouped_mm",
]
