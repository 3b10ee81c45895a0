"""Autograd functions of the MoE expert path (HIP kernels forward and backward).

The split follows the reference's module boundaries so each piece can be used
on its own:

  dispatch  (upstream dispatch, entered from npu_gmm.py:106-108)
      routed[j] = x[s_j // K] (* score[s_j] when score_before_experts)
  experts   (_run_experts_grouped_mm, npu_gmm.py:21-40)
      y = grouped_mm(swiglu(clamp(grouped_mm(routed, w13))), w2)
  combine   (upstream combine, npu_gmm.py:110)
      out[t] = sum_k (score[t,k] if score after experts else 1) * y[pos(t,k)]

plus the reference's own NPUMoeTokenUnpermute (npu_permute.py:15-53).
`moe_experts_forward` chains them; without autograd it takes the fused
route: the score multiply and the un-permute run in the w2 GEMM epilogue.
"""
from __future__ import annotations

import torch

from . import ops

_BF16 = torch.bfloat16


def _bf16(w: torch.Tensor) -> torch.Tensor:
    return w if w.dtype == _BF16 else w.to(_BF16)


class RouterFn(torch.autograd.Function):
    """Router forward (gate Linear in bf16 + fp32 softmax / sigmoid + top-k +
    renorm, UPSTREAM TokenChoiceTopKRouter; closed form
    torchtitanturbo/models/qwen3_5/model.py:752-766) with its backward on the
    HIP kernels: d(top_scores) -> d(logits) -> dx, dW_r.  The expert ids
    carry no gradient."""

    @staticmethod
    def forward(ctx, x, w_router, top_k, score_func, route_norm, route_scale, expert_bias, norm_eps):
        shape = x.shape
        xb = x.reshape(-1, shape[-1]).to(_BF16).contiguous()
        wb = _bf16(w_router).contiguous()
        scores, idx, logits = ops.router_fused(xb, wb, top_k, score_func, route_norm, route_scale, expert_bias,
                                               norm_eps, return_logits=True)
        ctx.save_for_backward(xb, wb, idx, logits)
        ctx.cfg = (score_func, route_norm, route_scale, norm_eps)
        ctx.x_shape, ctx.x_dtype, ctx.w_dtype = shape, x.dtype, w_router.dtype
        ctx.mark_non_differentiable(idx)
        return scores, idx

    @staticmethod
    def backward(ctx, g_scores, _g_idx):
        xb, wb, idx, logits = ctx.saved_tensors
        func, norm, scale, eps = ctx.cfg
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if g_scores is None or not (need_dx or need_dw):
            return (None,) * 8
        dx, dw = ops.router_backward(
            g_scores, idx, logits, xb, wb, func, norm, scale, eps, need_dx, need_dw,
            torch.float32 if ctx.w_dtype != _BF16 else _BF16,
        )
        if dx is not None:
            dx = dx.view(ctx.x_shape).to(ctx.x_dtype)
        if dw is not None:
            dw = dw.to(ctx.w_dtype)
        return dx, dw, None, None, None, None, None, None


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
    selected_experts_indices int64 [T, K]).  Differentiable in x and w_router
    when either requires grad (RouterFn), else the plain fused kernel."""
    if torch.is_grad_enabled() and (x.requires_grad or w_router.requires_grad):
        return RouterFn.apply(x, w_router, top_k, score_func, route_norm, route_scale, expert_bias, norm_eps)
    return ops.router_fused(x.reshape(-1, x.shape[-1]).to(_BF16), _bf16(w_router), top_k, score_func, route_norm,
                            route_scale, expert_bias, norm_eps)


class DispatchFn(torch.autograd.Function):
    """routed = gather of token rows in stable expert order (+ score before experts)."""

    @staticmethod
    def forward(ctx, x, scores_flat, sorted_indices, inverse, sorted_scores, top_k, score_before):
        ctx.top_k = top_k
        ctx.score_before = score_before
        if top_k == 1:
            routed = ops.gather_rows(x, sorted_indices, 1, sorted_scores if score_before else None)
        else:
            routed = ops.dispatch_rows(x, inverse, top_k, scores_flat if score_before else None)
        ctx.save_for_backward(x, scores_flat, sorted_indices, inverse)
        return routed

    @staticmethod
    def backward(ctx, d_routed):
        x, scores_flat, sorted_indices, inverse = ctx.saved_tensors
        d_routed = d_routed.to(_BF16).contiguous()
        dx = dscores = None
        probs = scores_flat if ctx.score_before else None
        if ctx.needs_input_grad[0]:
            dx = ops.combine(d_routed, inverse, probs, ctx.top_k)
        if ctx.score_before and ctx.needs_input_grad[1]:
            # d score[s] = <d_routed[pos(s)], x[s // K]>
            dscores = ops.rowdot_scatter(d_routed, x, sorted_indices, ctx.top_k)
        return dx, dscores, None, None, None, None, None


class ExpertsFn(torch.autograd.Function):
    """y = (swiglu(clamp(x @ w13[e]^T))) @ w2[e]^T over ragged expert groups."""

    @staticmethod
    def forward(ctx, routed, w13, w2, offs, swiglu_limit):
        w13b, w2b = _bf16(w13), _bf16(w2)
        # autograd runs forward() with grad mode off; needs_input_grad says
        # whether a backward can follow, i.e. whether h must be kept.
        need = any(ctx.needs_input_grad[:3])
        a, h = ops.grouped_mm_swiglu(routed, w13b, offs, swiglu_limit, save_h=need)
        y = ops.grouped_mm_unpermute(a, w2b, offs)
        ctx.swiglu_limit = swiglu_limit
        ctx.w_dtypes = (w13.dtype, w2.dtype)
        ctx.num_experts = w13.shape[0]
        if need:
            ctx.save_for_backward(routed, h, a, w13b, w2b, offs)
        return y

    @staticmethod
    def backward(ctx, dy):
        routed, h, a, w13b, w2b, offs = ctx.saved_tensors
        dy = dy.to(_BF16).contiguous()
        E = ctx.num_experts
        dh, _ = ops.grouped_mm_dgrad_swiglu(dy, w2b, h, offs, ctx.swiglu_limit)
        d_routed = dw13 = dw2 = None
        if ctx.needs_input_grad[2]:
            dw2 = ops.grouped_mm_wgrad(dy, a, offs, E, torch.float32 if ctx.w_dtypes[1] != _BF16 else _BF16)
            dw2 = dw2.to(ctx.w_dtypes[1])
        if ctx.needs_input_grad[1]:
            dw13 = ops.grouped_mm_wgrad(dh, routed, offs, E, torch.float32 if ctx.w_dtypes[0] != _BF16 else _BF16)
            dw13 = dw13.to(ctx.w_dtypes[0])
        if ctx.needs_input_grad[0]:
            d_routed = ops.grouped_mm_dgrad(dh, w13b, offs)
        return d_routed, dw13, dw2, None, None


class CombineFn(torch.autograd.Function):
    """out[t] = sum_k w(t,k) * y[pos(t,k)], w = score if score after experts else 1."""

    @staticmethod
    def forward(ctx, y, scores_flat, sorted_indices, inverse, top_k, score_after):
        ctx.top_k = top_k
        ctx.score_after = score_after
        probs = scores_flat if score_after else None
        out = ops.combine(y, inverse, probs, top_k)
        ctx.save_for_backward(y, scores_flat, sorted_indices)
        return out

    @staticmethod
    def backward(ctx, dout):
        y, scores_flat, sorted_indices = ctx.saved_tensors
        dout = dout.to(_BF16).contiguous()
        need_ds = ctx.score_after and ctx.needs_input_grad[1]
        dy, dscores = ops.token_unpermute_grad(
            dout, sorted_indices, scores_flat if ctx.score_after else None, y if need_ds else None,
            ctx.top_k, need_probs_grad=need_ds,
        )
        return dy, dscores, None, None, None, None


class HIPMoeTokenUnpermute(torch.autograd.Function):
    """Functional unpermute with backward; same contract as the reference's
    NPUMoeTokenUnpermute (torchtitanturbo/models/common/npu_permute.py:15-53):
    probs=None, top_k=1, empty input passes through.  With one choice per
    row and no probs the unpermute is a pure row scatter,
    out[sorted_indices[j]] = permuted_tokens[j], and its backward the
    matching gather, so both move rows bit for bit in the input's dtype."""

    @staticmethod
    def forward(ctx, permuted_tokens, sorted_indices, restore_shape):
        if not permuted_tokens.numel():
            return permuted_tokens
        rows = permuted_tokens.reshape(-1, permuted_tokens.shape[-1])
        out = ops.scatter_rows_exact(rows, sorted_indices.to(torch.int32))
        ctx.restore_shape = restore_shape
        ctx.save_for_backward(sorted_indices)
        return out.view(restore_shape)

    @staticmethod
    def backward(ctx, unpermuted_tokens_grad):
        if not unpermuted_tokens_grad.numel():
            return unpermuted_tokens_grad, None, None
        if ctx.needs_input_grad[0]:
            (sorted_indices,) = ctx.saved_tensors
            g = unpermuted_tokens_grad.reshape(-1, unpermuted_tokens_grad.shape[-1])
            act_grad = ops.gather_rows_exact(g, sorted_indices.to(torch.int32))
            return act_grad, None, None
        return None, None, None


class TokenPermuteFn(torch.autograd.Function):
    """permuted[j] = rows[sorted_indices[j]], sorted_indices the stable order of
    the row labels (torch_npu.npu_moe_token_permute with one label per row,
    npu_permute.py:74-76).  Rows move bit for bit in their own dtype; the
    backward scatters the gradient rows back, grad_rows[sorted_indices[j]] =
    grad_permuted[j] (npu_moe_token_permute's autograd)."""

    @staticmethod
    def forward(ctx, rows, labels, num_labels):
        r = ops.route(labels, num_labels)
        permuted = ops.gather_rows_exact(rows, r.sorted_indices)
        ctx.save_for_backward(r.sorted_indices)
        ctx.mark_non_differentiable(r.sorted_indices)
        return permuted, r.sorted_indices

    @staticmethod
    def backward(ctx, grad_permuted, _grad_idx):
        (sorted_indices,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        return ops.scatter_rows_exact(grad_permuted.contiguous(), sorted_indices), None, None


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
    y = ExpertsFn.apply(x.to(_BF16).contiguous(), w13, w2, offs, swiglu_limit)
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

    Without autograd this is one fused pass (ttamd_shared_expert_add: the
    shared w2 GEMM adds into the routed output in its epilogue).  With
    autograd it runs the shared FFN as a one-expert ExpertsFn and composes
    the gate and the sum in torch, so every input gets its gradient."""
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (routed_out, x, w13_shared, w2_shared, gate_logits))
    if not needs_grad:
        out = routed_out.to(_BF16).contiguous().clone()
        ops.shared_expert_add(out, x.to(_BF16), w13_shared, w2_shared,
                              None if gate_logits is None else gate_logits.float(), swiglu_limit)
        return out
    T = x.shape[0]
    all_rows = torch.full((1,), T, dtype=torch.int32, device=x.device)
    y = ExpertsFn.apply(x.to(_BF16).contiguous(), w13_shared.unsqueeze(0), w2_shared.unsqueeze(0), all_rows,
                        swiglu_limit)
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
    C-ABI call (ops.experts_forward: both grouped GEMMs on one tile table,
    the score multiply and the un-permute in the w2 GEMM epilogue).
    ``stage_events``, when given (inference path only), runs the same kernels
    one op at a time and receives a (start, end) pair of torch.cuda.Event
    per stage, recorded on the current stream around the stage's kernels:
    {"route", "permute", "gemm_w13_swiglu", "gemm_w2_unpermute", "sum_topk"}.
    """
    T, D = x.shape
    K = top_scores.shape[-1]
    training = torch.is_grad_enabled() and any(
        t.requires_grad for t in (x, top_scores, w13, w2)
    )
    ev = stage_events if (stage_events is not None and not training) else None

    def mark(name: str, end: bool) -> None:
        if ev is not None:
            pair = ev.setdefault(name, (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)))
            pair[1 if end else 0].record()

    scores_flat = top_scores.reshape(-1).float()
    mark("route", False)
    r = ops.route(selected_experts_indices, num_experts, scores_flat)
    mark("route", True)
    offs = r.offs
    xb = x.to(_BF16).contiguous()
    if not training and ev is None and D % 128 == 0:
        out = ops.experts_forward(xb, r, _bf16(w13), _bf16(w2), K, score_before_experts, swiglu_limit)
        return out.to(x.dtype)
    if not training:
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
    routed = DispatchFn.apply(
        xb, scores_flat, r.sorted_indices, r.inverse, r.sorted_scores, K, score_before_experts
    )
    y = ExpertsFn.apply(routed, w13, w2, offs, swiglu_limit)
    out = CombineFn.apply(y, scores_flat, r.sorted_indices, r.inverse, K, not score_before_experts)
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
