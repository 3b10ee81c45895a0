"""The inference MoE layer forward captured as one HIP graph.

A step of the layer is two C-ABI calls (ttamd_router_route, then
ttamd_moe_experts_forward: six kernel launches, all on the caller's
stream, none of them a memset, a host synchronisation or an allocation
inside the library).  At small shapes the host's cost per call exceeds
the kernels' run time (T = 2048, D = 256), so the pair
is recorded once with torch's graph capture over that stream and replayed:
one launch per step.  Every buffer the step uses (the routing outputs, the
tile plan, the workspaces, the output) is allocated once, during capture,
from the graph's private pool.

Reference: the step is NpuGroupedExperts.forward with its router
(torchtitanturbo/models/common/npu_gmm.py:100-110; router closed form
models/qwen3_5/model.py:752-766), inference only.
"""
from __future__ import annotations

import torch

from . import ops

_BF16 = torch.bfloat16


class MoELayerGraph:
    """Router + dispatch + experts + combine for a fixed [T, D] input shape,
    captured once and replayed.

    ``layer(x)`` copies x into the graph's input buffer, replays the graph
    on the current stream and returns the graph's output buffer: the next
    call overwrites it, so clone it to keep it.  Weights are read where they
    are at capture time (update them in place, not by rebinding).
    """

    def __init__(
        self,
        x: torch.Tensor,
        w_router: torch.Tensor,
        w13: torch.Tensor,
        w2: torch.Tensor,
        top_k: int,
        score_func: str = "softmax",
        route_norm: bool = False,
        score_before_experts: bool = False,
        route_scale: float = 1.0,
        expert_bias: torch.Tensor | None = None,
        swiglu_limit: float | None = None,
        warmup: int = 2,
    ):
        if x.dim() != 2 or x.dtype != _BF16:
            raise TypeError("x must be a bf16 [T, D] tensor")
        for name, t in (("w_router", w_router), ("w13", w13), ("w2", w2)):
            if t.dtype != _BF16 or not t.is_contiguous():
                raise TypeError(f"{name} must be a contiguous bf16 tensor (read in place by the graph)")
        self._args = (w_router, w13, w2, top_k, score_func, route_norm, score_before_experts, route_scale,
                      expert_bias, swiglu_limit)
        self.static_x = x.detach().clone()
        # warm up on a side stream (first calls set kernel attributes), then capture
        side = torch.cuda.Stream(device=x.device)
        side.wait_stream(torch.cuda.current_stream(x.device))
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(warmup):
                self._step(self.static_x)
        torch.cuda.current_stream(x.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.static_out = self._step(self.static_x)

    def _step(self, x: torch.Tensor) -> torch.Tensor:
        w_router, w13, w2, top_k, func, norm, before, scale, bias, limit = self._args
        _, _, r = ops.router_route(x, w_router, top_k, func, norm, scale, bias, with_inverse=False)
        return ops.experts_forward(x, r, w13, w2, top_k, before, limit)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape != self.static_x.shape:
            raise ValueError(f"captured for x {tuple(self.static_x.shape)}, got {tuple(x.shape)}")
        self.static_x.copy_(x)
        self.graph.replay()
        return self.static_out

    def replay(self) -> torch.Tensor:
        """Replay on the input already in ``static_x``."""
        self.graph.replay()
        return self.static_out
