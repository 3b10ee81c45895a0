"""Autograd-carrying functions of the MoE expert path (HIP kernels forward
and backward), built on the registered ``ttamd::*`` custom ops of
``library.py`` so that torch.compile / AOTAutograd trace them as opaque
nodes with their registered backward.

The split follows the reference's module boundaries so each piece can be used
on its own:

  router    (UPSTREAM TokenChoiceTopKRouter; closed form qwen3_5/model.py:752-766)
  dispatch  (upstream dispatch, entered from npu_gmm.py:106-108)
      routed[j] = x[s_j // K] (* score[s_j] when score_before_experts)
  experts   (_run_experts_grouped_mm, npu_gmm.py:21-40)
      y = grouped_mm(swiglu(clamp(grouped_mm(routed, w13))), w2)
  combine   (upstream combine, npu_gmm.py:110)
      out[t] = sum_k (score[t,k] if score after experts else 1) * y[pos(t,k)]

plus the reference's own NPUMoeTokenUnpermute (npu_permute.py:15-53).
`moe_experts_forward` chains them; without autograd it takes the fused
inference op (one C-ABI call for the whole expert stage).
"""
from __future__ import annotations

import torch

from . import library  # noqa: F401  (registers the ttamd::* ops)
from . import ops

_BF16 = torch.bfloat16
_T = torch.ops.ttamd


def _bf16(w: torch.Tensor) -> torch.Tensor:
    return library._bf(w)


def _needs_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def router(
    x: torch.Tensor,
    w_router: torch.Tensor,
    top_k: int,
    score_func: str = "softmax",
    route_norm: bool = False,
    route_scale: float = 1.0,
    expert_bias: torch.Tensor | None = None,
    norm_eps: float = 1e-20,
) -> tuple[torch.Tensor, torch.Tensor]:
    """UPSTREAM TokenChoiceTopKRouter forward: (top_scores fp32 [T, K],
    selected_experts_indices int64 [T, K]).  x [..., D] and w_router [E, D]
    in any float dtype (bf16 inside the op, so their gradients come back in
    their own dtype); differentiable in x and w_router through ttamd::router's
    registered backward, the expert ids carry no gradient."""
    xb = x.reshape(-1, x.shape[-1]).to(_BF16).contiguous()
    scores, idx, _ = _T.router(xb, w_router, top_k, score_func, route_norm, route_scale, expert_bias, norm_eps)
    return scores, idx


def dispatch(x, scores_flat, sorted_indices, inverse, sorted_scores, top_k, score_before):
    """routed = gather of token rows in stable expert order (+ score before experts)."""
    return _T.dispatch(x, scores_flat, sorted_indices, inverse, sorted_scores, top_k, score_before)


def experts(routed, w13, w2, offs, swiglu_limit):
    """y = (swiglu(clamp(x @ w13[e]^T))) @ w2[e]^T over ragged expert groups;
    the pre-activation, the SwiGLU output and (for weights that are not bf16)
    the forward's bf16 weight copies are kept only when a backward can
    follow."""
    keep = _needs_grad(routed, w13, w2)
    return _T.experts(routed, w13, w2, offs, swiglu_limit, keep)[0]


def combine(y, scores_flat, sorted_indices, inverse, top_k, score_after):
    """out[t] = sum_k w(t,k) * y[pos(t,k)], w = score if score after experts else 1."""
    return _T.combine(y, scores_flat, sorted_indices, inverse, top_k, score_after)


class HIPMoeTokenUnpermute:
    """Functional unpermute with backward; same contract as the reference's
    NPUMoeTokenUnpermute (torchtitanturbo/models/common/npu_permute.py:15-53):
    probs=None, top_k=1, empty input passes through.  With one choice per
    row and no probs the unpermute is a pure row scatter,
    out[sorted_indices[j]] = permuted_tokens[j], and its backward the
    matching gather (ttamd::token_unpermute), so both move rows bit for bit
    in the input's dtype."""

    @staticmethod
    def apply(permuted_tokens, sorted_indices, restore_shape):
        if not permuted_tokens.numel():
            return permuted_tokens
        rows = permuted_tokens.reshape(-1, permuted_tokens.shape[-1])
        return _T.token_unpermute(rows, sorted_indices).view(restore_shape)


def token_permute(rows, labels, num_labels):
    """permuted[j] = rows[sorted_indices[j]], sorted_indices the stable order of
    the row labels (torch_npu.npu_moe_token_permute with one label per row,
    npu_permute.py:74-76).  Rows move bit for bit in their own dtype; the
    backward scatters the gradient rows back, grad_rows[sorted_indices[j]] =
    grad_permuted[j] (ttamd::token_permute)."""
    return _T.token_permute(rows, labels, num_labels)


def run_experts_grouped_mm(
    w13: torch.Tensor,
    w2: torch.Tensor,
    x: torch.Tensor,
    num_tokens_per_expert: torch.Tensor,
    swiglu_limit: float | None = None,
) -> torch.Tensor:
    """Same signature and result as the reference's _run_experts_grouped_mm
    (torchtitanturbo/models/common/npu_gmm.py:21-40), on the HIP kernels."""
    offs = torch.cumsum(num_tokens_per_expert, dim=0, dtype=torch.int32)
    y = experts(x.to(_BF16).contiguous(), w13, w2, offs, swiglu_limit)
    return y.type_as(x)


def shared_expert_combine(
    routed_out: torch.Tensor,
    x: torch.Tensor,
    w13_shared: torch.Tensor,
    w2_shared: torch.Tensor,
    gate_logits: torch.Tensor | None = None,
    swiglu_limit: float | None = None,
) -> torch.Tensor:
    """routed_out + g * shared_expert(x), g = sigmoid(gate_logits) or 1
    (torchtitanturbo/models/qwen3_5/model.py:796-809; UPSTREAM Llama4 adds the
    ungated shared expert).  x [T, D]; w13_shared [2H, D]; w2_shared [D, H].

    Without autograd this is one fused pass (ttamd::shared_expert_add: the
    shared w2 GEMM adds into the routed output in its epilogue).  With
    autograd it runs the shared FFN as a one-expert ttamd::experts and
    composes the gate and the sum in torch, so every input gets its
    gradient."""
    if not _needs_grad(routed_out, x, w13_shared, w2_shared, gate_logits):
        return _T.shared_expert_add(routed_out, x, w13_shared, w2_shared, gate_logits, swiglu_limit)
    T = x.shape[0]
    all_rows = torch.full((1,), T, dtype=torch.int32, device=x.device)
    y = experts(x.to(_BF16).contiguous(), w13_shared.unsqueeze(0), w2_shared.unsqueeze(0), all_rows, swiglu_limit)
    if gate_logits is not None:
        y = torch.sigmoid(gate_logits.to(y.dtype)).reshape(T, 1) * y
    return routed_out + y


def moe_experts_forward(
    x: torch.Tensor,
    top_scores: torch.Tensor,
    selected_experts_indices: torch.Tensor,
    w13: torch.Tensor,
    w2: torch.Tensor,
    num_experts: int,
    score_before_experts: bool,
    swiglu_limit: float | None = None,
    stage_events: dict | None = None,
) -> torch.Tensor:
    """dispatch -> experts -> combine for one GPU; x [T, D], scores/indices [T, K] -> [T, D].

    With autograd off (or nothing requiring grad) the expert stage is one
    op (ttamd::moe_experts_forward: both grouped GEMMs on one tile table,
    the score multiply and the un-permute in the w2 GEMM epilogue).
    ``stage_events``, when given (inference path only), runs the same kernels
    one op at a time and receives a (start, end) pair of torch.cuda.Event
    per stage, recorded on the current stream around the stage's kernels:
    {"route", "permute", "gemm_w13_swiglu", "gemm_w2_unpermute", "sum_topk"}.
    """
    T, D = x.shape
    K = top_scores.shape[-1]
    training = _needs_grad(x, top_scores, w13, w2)
    ev = stage_events if (stage_events is not None and not training) else None

    def mark(name: str, end: bool) -> None:
        if ev is not None:
            pair = ev.setdefault(name, (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)))
            pair[1 if end else 0].record()

    scores_flat = top_scores.reshape(-1).float()
    mark("route", False)
    counts, offsets, sorted_idx, inverse, sorted_scores = _T.route(
        selected_experts_indices.reshape(-1), num_experts, scores_flat.detach())
    mark("route", True)
    offs = offsets[1:]
    xb = x.to(_BF16).contiguous()
    if not training and ev is None and D % 128 == 0:
        out = _T.moe_experts_forward(xb, sorted_idx, offsets, sorted_scores, _bf16(w13), _bf16(w2), K,
                                     score_before_experts, swiglu_limit)
        return out.to(x.dtype)
    if not training:
        # op-at-a-time over the same kernels (stage timing; D < 128)
        r = ops.RouteResult(counts, offsets, sorted_idx, inverse, sorted_scores)
        w13b, w2b = _bf16(w13), _bf16(w2)
        if score_before_experts or D < 128:
            mark("permute", False)
            routed = ops.permute_rows(xb, r, K, scores_flat if score_before_experts else None)
            mark("permute", True)
            mark("gemm_w13_swiglu", False)
            a, _ = ops.grouped_mm_swiglu(routed, w13b, offs, swiglu_limit)
            mark("gemm_w13_swiglu", True)
        else:
            # the permute gather happens inside the w13 GEMM's loads
            mark("gemm_w13_swiglu", False)
            a, _ = ops.grouped_mm_swiglu_gather(xb, r.sorted_indices, K, w13b, offs, swiglu_limit)
            mark("gemm_w13_swiglu", True)
        scale = None if score_before_experts else r.sorted_scores
        if K == 1:
            mark("gemm_w2_unpermute", False)
            out = ops.grouped_mm_unpermute(a, w2b, offs, scale, r.sorted_indices, T)
            mark("gemm_w2_unpermute", True)
        else:
            mark("gemm_w2_unpermute", False)
            ybuf = ops.grouped_mm_unpermute(a, w2b, offs, scale, r.sorted_indices, T * K)
            mark("gemm_w2_unpermute", True)
            mark("sum_topk", False)
            out = ops.sum_topk(ybuf, K)
            mark("sum_topk", True)
        return out.to(x.dtype)
    routed = dispatch(xb, scores_flat, sorted_idx, inverse, sorted_scores, K, score_before_experts)
    y = experts(routed, w13, w2, offs, swiglu_limit)
    out = combine(y, scores_flat, sorted_idx, inverse, K, not score_before_experts)
    return out.to(x.dtype)


def moe_experts_forward_fp8(
    x: torch.Tensor,
    top_scores: torch.Tensor,
    selected_experts_indices: torch.Tensor,
    w13q: torch.Tensor,
    s13: torch.Tensor,
    w2q: torch.Tensor,
    s2: torch.Tensor,
    num_experts: int,
    score_before_experts: bool,
    swiglu_limit: float | None = None,
    stage_events: dict | None = None,
) -> torch.Tensor:
    """Inference forward with fp8 e4m3 experts (weights pre-quantised with
    ops.quantize_fp8_blocks): route -> gather + per-token quantise -> fp8
    w13 + SwiGLU -> per-token re-quantise of a -> fp8 w2 + scale + scatter
    -> K-way sum.  x [T, D] bf16 -> [T, D]."""
    T, D = x.shape
    K = top_scores.shape[-1]
    ev = stage_events

    def mark(name: str, end: bool) -> None:
        if ev is not None:
            pair = ev.setdefault(name, (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)))
            pair[1 if end else 0].record()

    scores_flat = top_scores.reshape(-1).float()
    mark("route", False)
    r = ops.route(selected_experts_indices, num_experts, scores_flat)
    mark("route", True)
    xb = x.to(_BF16).contiguous()
    mark("permute_quantize", False)
    xq, sx = ops.quantize_fp8_rows(xb, r.sorted_indices, K, r.sorted_scores if score_before_experts else None)
    mark("permute_quantize", True)
    mark("gemm_w13_swiglu", False)
    a, _ = ops.grouped_mm_fp8_swiglu(xq, sx, w13q, s13, r.offs, swiglu_limit)
    mark("gemm_w13_swiglu", True)
    mark("quantize_a", False)
    aq, sa = ops.quantize_fp8_rows(a)
    mark("quantize_a", True)
    scale = None if score_before_experts else r.sorted_scores
    mark("gemm_w2_unpermute", False)
    if K == 1:
        out = ops.grouped_mm_fp8_unpermute(aq, sa, w2q, s2, r.offs, scale, r.sorted_indices, T)
        mark("gemm_w2_unpermute", True)
    else:
        ybuf = ops.grouped_mm_fp8_unpermute(aq, sa, w2q, s2, r.offs, scale, r.sorted_indices, T * K)
        mark("gemm_w2_unpermute", True)
        mark("sum_topk", False)
        out = ops.sum_topk(ybuf, K)
        mark("sum_topk", True)
    return out.to(x.dtype)
