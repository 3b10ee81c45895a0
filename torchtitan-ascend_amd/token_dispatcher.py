"""HipTokenDispatcher and its converter: the token side of the MoE expert path.

Mirrors torchtitanturbo/models/common/npu_permute.py:
  * HipTokenDispatcher            <- NpuTokenDispatcher (:56-88)
  * HIPMoeTokenUnpermute          <- NPUMoeTokenUnpermute (:15-53)
  * HipTokenDispatcherConverter   <- NpuTokenDispatcherConverter (:91-117)

On one GPU (no expert-parallel mesh) `dispatch`/`combine` run the whole
local dispatch on the HIP routing kernels: histogram, stable counting sort,
row gather with the optional score multiply, and the deterministic K-way
gather-sum.  `_permute`/`_unpermute` are the expert-parallel regroup
(rank-major -> expert-major) of the reference; they are usable on one GPU
with synthetic per-(rank, expert) counts.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from . import functional as Fn
from .functional import HIPMoeTokenUnpermute
from .protocol import AllToAllTokenDispatcher, GroupedExperts, ModelConfigConverter


@dataclass
class HipDispatchMetadata:
    """What combine needs from dispatch (all device tensors)."""

    sorted_indices: torch.Tensor  # int32 [M]
    inverse: torch.Tensor  # int32 [M]
    scores_flat: torch.Tensor  # fp32 [M] (autograd-connected to top_scores)
    offsets: torch.Tensor  # int32 [E+1] exclusive
    num_tokens: int
    top_k: int


# Attributes under which an expert-parallel setup may attach its device mesh
# or process group to the dispatcher module.
_EP_ATTRS = ("ep_mesh", "device_mesh", "mesh", "ep_group", "process_group", "group")


def _group_size(obj) -> int:
    """Ranks of a DeviceMesh / ProcessGroup-like object (its size())."""
    size = getattr(obj, "size", None)
    if callable(size):
        return int(size())
    raise RuntimeError(f"HipTokenDispatcher: cannot read the size of the attached {type(obj).__name__}")


class HipTokenDispatcher(AllToAllTokenDispatcher):
    """Token dispatcher on hand-written MI355X routing kernels."""

    @dataclass(kw_only=True, slots=True)
    class Config(AllToAllTokenDispatcher.Config):
        # Expert-parallel degree when it is known from outside (None: read it
        # from an attached mesh, else from torch.distributed's world size).
        expert_parallel_degree: int | None = None

    def __init__(self, config: "HipTokenDispatcher.Config"):
        super().__init__(config)
        self.num_experts = config.num_experts
        self.top_k = config.top_k
        self.score_before_experts = config.score_before_experts
        self.expert_parallel_degree = config.expert_parallel_degree

    @property
    def is_local(self) -> bool:
        """True only when the expert-parallel degree is provably 1: every
        mesh or process group attached to the module has one rank, or the
        config declares degree 1, or torch.distributed runs a single rank
        (or none).  False when a larger mesh is attached or degree > 1 is
        declared (dispatch then refuses: no all-to-all in this build).
        Raises when torch.distributed runs several ranks and nothing says
        how many of them share the experts, so that a shard never takes the
        single-GPU path by accident."""
        sizes = {n: _group_size(m) for n in _EP_ATTRS if (m := getattr(self, n, None)) is not None}
        if sizes:
            return all(v == 1 for v in sizes.values())
        if self.expert_parallel_degree is not None:
            return int(self.expert_parallel_degree) == 1
        dist = torch.distributed
        if not dist.is_available() or not dist.is_initialized() or dist.get_world_size() == 1:
            return True
        raise RuntimeError(
            f"HipTokenDispatcher: torch.distributed runs {dist.get_world_size()} ranks and no expert-parallel "
            f"mesh is attached (looked for {', '.join(_EP_ATTRS)}); set expert_parallel_degree in "
            "HipTokenDispatcher.Config (1 for data parallelism only)"
        )

    def dispatch(self, x, top_scores, selected_experts_indices):
        """x [T, D], top_scores / selected_experts_indices [T, K] ->
        (routed_input [T*K, D], num_tokens_per_expert int32 [E], metadata)."""
        if not self.is_local:
            raise NotImplementedError("expert-parallel all-to-all (degree > 1) is not part of this single-GPU build")
        T, _ = x.shape
        K = top_scores.shape[-1]
        scores_flat = top_scores.reshape(-1).float()
        r = ops.route(selected_experts_indices, self.num_experts, scores_flat)
        routed = Fn.dispatch(
            x.to(torch.bfloat16).contiguous(), scores_flat, r.sorted_indices, r.inverse, r.sorted_scores, K,
            self.score_before_experts,
        )
        meta = HipDispatchMetadata(r.sorted_indices, r.inverse, scores_flat, r.offsets, T, K)
        return routed, r.counts, meta

    def combine(self, routed_output, metadata: HipDispatchMetadata, x):
        """routed_output [T*K, D] in dispatch order -> [T, D] in x's dtype."""
        out = Fn.combine(
            routed_output.to(torch.bfloat16).contiguous(), metadata.scores_flat, metadata.sorted_indices,
            metadata.inverse, metadata.top_k, not self.score_before_experts,
        )
        return out.to(x.dtype)

    def _permute(self, routed_input, num_tokens_per_expert_group, ep_size, num_local_experts):
        """Regroup rows received rank-major (rank, expert) into expert-major order.

        Same contract as NpuTokenDispatcher._permute (npu_permute.py:63-85):
        returns (input_shape, permuted_input, permuted_indices, num_tokens_per_expert).
        """
        labels = ops.group_labels(num_tokens_per_expert_group, num_local_experts, routed_input.shape[0])
        # rows move bit for bit in routed_input's dtype, with autograd (the
        # backward scatters the gradient rows back)
        permuted, permuted_indices = Fn.token_permute(routed_input, labels, num_local_experts)
        num_tokens_per_expert = num_tokens_per_expert_group.view(ep_size, -1).sum(0)
        return routed_input.shape, permuted, permuted_indices, num_tokens_per_expert

    def _unpermute(self, routed_output, input_shape, permuted_indices):
        return HIPMoeTokenUnpermute.apply(routed_output, permuted_indices, input_shape)


def _experts_configs(model_config):
    """Every experts config that carries a token dispatcher, converted or not
    (the reference only looks at GroupedExperts.Config, so running its
    dispatcher converter after its experts converter finds nothing)."""
    from .grouped_experts import HipGroupedExperts

    seen = set()
    for cls in (GroupedExperts.Config, HipGroupedExperts.Config):
        for fqn, cfg, parent, attr in model_config.traverse(cls):
            if id(cfg) not in seen:
                seen.add(id(cfg))
                yield fqn, cfg, parent, attr


class HipTokenDispatcherConverter(ModelConfigConverter):
    """Replace AllToAllTokenDispatcher configs with HipTokenDispatcher configs."""

    @dataclass(kw_only=True, slots=True)
    class Config(ModelConfigConverter.Config):
        # passed to every converted dispatcher (None: found at run time)
        expert_parallel_degree: int | None = None

    def __init__(self, config: "HipTokenDispatcherConverter.Config"):
        self.config = config

    def convert(self, model_config) -> None:
        count = 0
        for _fqn, cfg, _parent, _attr in _experts_configs(model_config):
            td = cfg.token_dispatcher
            if isinstance(td, AllToAllTokenDispatcher.Config) and not isinstance(td, HipTokenDispatcher.Config):
                cfg.token_dispatcher = HipTokenDispatcher.Config(
                    num_experts=td.num_experts,
                    top_k=td.top_k,
                    score_before_experts=td.score_before_experts,
                    expert_parallel_degree=self.config.expert_parallel_degree,
                )
                count += 1
        self.num_converted = count
