"""The reference path's own op sequence on the CPU, in torch -- BASELINE AND
TEST INFRASTRUCTURE ONLY.

bench.py's cpu_baseline leg times this on the GPU box's host cores, and
tests/test_reference_cpu.py checks it against the numpy oracle
(moe_oracle.py).  Nothing in the product imports it.

The reference (torchtitanturbo) cannot run here: its hot-path modules import
torch_npu and torchtitan at top level (npu_gmm.py:7-14, npu_permute.py:6-12),
neither of which exists in this image.  This module restates the same op
sequence with each closed torch_npu op replaced by the torch op whose
closed form it computes:

  router      models/qwen3_5/model.py:752-766 (UPSTREAM TokenChoiceTopKRouter):
              F.linear in bf16, softmax / sigmoid in fp32, torch.topk, renorm
  dispatch    UPSTREAM dispatch reached from npu_gmm.py:106-108, and
              npu_moe_token_permute (npu_permute.py:74-76): histc counts,
              stable argsort of the flat labels, index_select of the rows
              (* score in fp32 when score_before_experts)
  experts     _run_experts_grouped_mm (npu_gmm.py:21-40): cumsum offsets,
              torch._grouped_mm bf16 for w13, optional clamp, npu_swiglu ->
              silu(gate) * up, torch._grouped_mm bf16 for w2
  combine     UPSTREAM combine reached from npu_gmm.py:110: score multiply
              after the experts, scatter back to the flat slots, sum over K
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def router(x: torch.Tensor, w_router: torch.Tensor, top_k: int, score_func: str = "softmax",
           route_norm: bool = False, eps: float = 1e-20):
    """Top-k router: returns (top_scores fp32 [T, K], indices int64 [T, K])."""
    logits = F.linear(x, w_router)  # bf16 gate (model.py:757)
    if score_func == "softmax":
        scores = torch.softmax(logits.float(), dim=-1)  # (:758)
    else:
        scores = torch.sigmoid(logits.float())
    top_scores, idx = torch.topk(scores, top_k, dim=-1)  # (:759-761)
    if route_norm:
        top_scores = top_scores / (top_scores.sum(dim=-1, keepdim=True) + eps)  # (:762-764)
    return top_scores, idx


def moe_layer(x: torch.Tensor, top_scores: torch.Tensor, idx: torch.Tensor, w13: torch.Tensor,
              w2: torch.Tensor, num_experts: int, score_before_experts: bool,
              swiglu_limit: float | None = None) -> torch.Tensor:
    """dispatch -> experts -> combine; x [T, D] bf16, w13 [E, 2H, D], w2 [E, D, H] -> [T, D] bf16."""
    T, D = x.shape
    K = idx.shape[-1]
    flat = idx.reshape(-1)
    counts = torch.histc(flat.float(), bins=num_experts, min=0, max=num_experts)
    order = torch.argsort(flat, stable=True)
    scores_sorted = top_scores.reshape(-1).float()[order]
    routed = x.index_select(0, order // K)
    if score_before_experts:
        routed = (routed.float() * scores_sorted[:, None]).to(x.dtype)
    offs = torch.cumsum(counts, dim=0).to(torch.int32)  # npu_gmm.py:29
    h = torch._grouped_mm(routed.bfloat16(), w13.bfloat16().transpose(-2, -1), offs=offs)  # :31
    H = h.shape[-1] // 2
    gate, up = h[:, :H], h[:, H:]
    if swiglu_limit is not None:  # :32-36
        gate = gate.clamp(max=swiglu_limit)
        up = up.clamp(min=-swiglu_limit, max=swiglu_limit)
    a = F.silu(gate) * up  # npu_swiglu (:37)
    y = torch._grouped_mm(a, w2.bfloat16().transpose(-2, -1), offs=offs).type_as(x)  # :38
    if not score_before_experts:
        y = (y.float() * scores_sorted[:, None]).to(x.dtype)
    out = torch.zeros(T * K, D, dtype=y.dtype)
    out[order] = y
    return out.view(T, K, D).sum(dim=1)


def moe_step(x, w_router, w13, w2, num_experts, top_k, score_func, route_norm, score_before_experts,
             labels=None, label_scores=None, swiglu_limit=None, shared=None):
    """One step of the bench workload: router (or given labels and scores)
    then the layer; `shared` = (w13_shared [2H, D], w2_shared [D, H]) adds
    the always-on shared expert (a one-expert grouped GEMM on every token)."""
    if labels is None:
        top_scores, idx = router(x, w_router, top_k, score_func, route_norm)
    else:
        top_scores, idx = label_scores, labels
    out = moe_layer(x, top_scores, idx, w13, w2, num_experts, score_before_experts, swiglu_limit)
    if shared is not None:
        T = x.shape[0]
        ones = torch.ones(T, 1, dtype=torch.float32)
        zeros = torch.zeros(T, 1, dtype=torch.int64)
        out = out + moe_layer(x, ones, zeros, shared[0][None], shared[1][None], 1, True, swiglu_limit)
    return out
