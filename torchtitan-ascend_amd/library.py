"""torch.library custom ops of the MoE expert path (namespace ``ttamd``).

Every device step of the path is one registered op, with a fake (meta)
implementation for shape propagation and, where the reference's autograd
reaches it, a registered backward that is itself a registered op.  The ops
are therefore traceable: torch.compile / AOTAutograd see opaque ``ttamd::*``
nodes instead of breaking the graph at a ctypes call, and
``torch.library.opcheck`` can check each registration.  The implementations
call the C ABI through ``ops``; they are registered for every device so that
a tensor off the GPU reaches ``ops`` and gets its RuntimeError (the path has
no CPU or eager-torch fallback).

Reference ops these stand for (torchtitanturbo/models/common/):
  * ttamd::router / router_backward   UPSTREAM TokenChoiceTopKRouter
                                      (closed form qwen3_5/model.py:752-766)
  * ttamd::route                      histc + stable argsort of dispatch
                                      (npu_gmm.py:106-108)
  * ttamd::dispatch (+ backward)      dispatch gather / score-before
  * ttamd::experts (+ backward)       _run_experts_grouped_mm, npu_gmm.py:21-40
  * ttamd::combine (+ backward)       combine / NPUMoeTokenUnpermute, npu_permute.py:15-53
  * ttamd::moe_experts_forward        the fused inference expert stage
  * ttamd::shared_expert_add          shared-expert tail, qwen3_5/model.py:796-809
  * ttamd::token_permute / token_unpermute (+ backward)
                                      npu_moe_token_permute / unpermute, npu_permute.py:74-88
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import ops

_BF16 = torch.bfloat16
_F32 = torch.float32
_I32 = torch.int32


def _empty(t: Tensor) -> Tensor:
    return t.new_empty((0,))


def _bf(w: Tensor) -> Tensor:
    """bf16 copy of a weight that is not bf16 (the per-call .bfloat16() of
    npu_gmm.py:31, :38): torch's device cast, one streaming pass at
    ~5.9 TB/s on MI355X."""
    return w if w.dtype == _BF16 else w.to(_BF16)


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::router", mutates_args=())
def router(x: Tensor, w_router: Tensor, top_k: int, score_func: str, route_norm: bool, route_scale: float,
           expert_bias: Optional[Tensor], norm_eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """x bf16 [T, D], w_router [E, D] (bf16, or fp32 master weights used in
    bf16 as the gate Linear sees them) -> (top_scores fp32 [T, K],
    selected_experts_indices int64 [T, K], logits bf16 [T, E])."""
    return ops.router_fused(x, _bf(w_router), top_k, score_func, route_norm, route_scale, expert_bias, norm_eps,
                            return_logits=True)


@router.register_fake
def _(x, w_router, top_k, score_func, route_norm, route_scale, expert_bias, norm_eps):
    T, E = x.shape[0], w_router.shape[0]
    return (x.new_empty((T, top_k), dtype=_F32), x.new_empty((T, top_k), dtype=torch.int64),
            x.new_empty((T, E), dtype=_BF16))


@torch.library.custom_op("ttamd::router_backward", mutates_args=())
def router_backward(grad_scores: Tensor, idx: Tensor, logits: Tensor, x: Tensor, w_router: Tensor, score_func: str,
                    route_norm: bool, route_scale: float, norm_eps: float) -> tuple[Tensor, Tensor]:
    """(dx bf16 [T, D], dW_r [E, D] in w_router's dtype: an fp32 weight gets
    the fp32 sums of the wgrad kernel, unrounded) from d(top_scores) [T, K]."""
    dx, dw = ops.router_backward(grad_scores, idx, logits, x, _bf(w_router), score_func, route_norm, route_scale,
                                 norm_eps, True, True, _F32 if w_router.dtype != _BF16 else _BF16)
    return dx, dw.to(w_router.dtype)


@router_backward.register_fake
def _(grad_scores, idx, logits, x, w_router, score_func, route_norm, route_scale, norm_eps):
    return x.new_empty(x.shape, dtype=_BF16), w_router.new_empty(w_router.shape)


def _router_setup(ctx, inputs, output):
    x, w_router, _k, func, norm, scale, _bias, eps = inputs
    _, idx, logits = output
    ctx.save_for_backward(x, w_router, idx, logits)
    ctx.cfg = (func, norm, scale, eps)
    # the logits are returned for the backward only: no zero gradient for them
    ctx.set_materialize_grads(False)


def _router_bwd(ctx, g_scores, _g_idx, _g_logits):
    if g_scores is None:
        return None, None, None, None, None, None, None, None
    x, w_router, idx, logits = ctx.saved_tensors
    func, norm, scale, eps = ctx.cfg
    dx, dw = router_backward(g_scores.contiguous(), idx, logits, x, w_router, func, norm, scale, eps)
    return dx, dw, None, None, None, None, None, None


router.register_autograd(_router_bwd, setup_context=_router_setup)


# ---------------------------------------------------------------------------
# Route (no gradient: integer order + a gathered copy of the scores)
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::route", mutates_args=())
def route(idx: Tensor, num_experts: int, scores: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(counts int32 [E], offsets int32 [E + 1], sorted_indices int32 [M],
    inverse int32 [M], sorted_scores fp32 [M]) of the flat labels idx."""
    r = ops.route(idx, num_experts, scores)
    return r.counts, r.offsets, r.sorted_indices, r.inverse, r.sorted_scores


@route.register_fake
def _(idx, num_experts, scores):
    M = idx.numel()
    return (idx.new_empty((num_experts,), dtype=_I32), idx.new_empty((num_experts + 1,), dtype=_I32),
            idx.new_empty((M,), dtype=_I32), idx.new_empty((M,), dtype=_I32), idx.new_empty((M,), dtype=_F32))


# ---------------------------------------------------------------------------
# Dispatch: routed[j] = x[s_j // K] (* score[s_j] before the experts)
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::dispatch", mutates_args=())
def dispatch(x: Tensor, scores_flat: Tensor, sorted_indices: Tensor, inverse: Tensor, sorted_scores: Tensor,
             top_k: int, score_before: bool) -> Tensor:
    if top_k == 1:
        return ops.gather_rows(x, sorted_indices, 1, sorted_scores if score_before else None)
    return ops.dispatch_rows(x, inverse, top_k, scores_flat if score_before else None)


@dispatch.register_fake
def _(x, scores_flat, sorted_indices, inverse, sorted_scores, top_k, score_before):
    return x.new_empty((sorted_indices.numel(), x.shape[1]))


@torch.library.custom_op("ttamd::dispatch_backward", mutates_args=())
def dispatch_backward(d_routed: Tensor, x: Tensor, scores_flat: Tensor, sorted_indices: Tensor, inverse: Tensor,
                      top_k: int, score_before: bool) -> tuple[Tensor, Tensor]:
    """(dx [T, D], d scores_flat [M] (empty unless score_before))."""
    d_routed = d_routed.to(_BF16).contiguous()
    dx = ops.combine(d_routed, inverse, scores_flat if score_before else None, top_k)
    # d score[s] = <d_routed[pos(s)], x[s // K]>
    ds = ops.rowdot_scatter(d_routed, x, sorted_indices, top_k) if score_before else _empty(scores_flat)
    return dx, ds


@dispatch_backward.register_fake
def _(d_routed, x, scores_flat, sorted_indices, inverse, top_k, score_before):
    return x.new_empty(x.shape), scores_flat.new_empty(scores_flat.shape if score_before else (0,))


def _dispatch_setup(ctx, inputs, output):
    x, scores_flat, sorted_indices, inverse, _ss, top_k, score_before = inputs
    ctx.save_for_backward(x, scores_flat, sorted_indices, inverse)
    ctx.cfg = (top_k, score_before)


def _dispatch_bwd(ctx, d_routed):
    x, scores_flat, sorted_indices, inverse = ctx.saved_tensors
    top_k, score_before = ctx.cfg
    dx, ds = dispatch_backward(d_routed, x, scores_flat, sorted_indices, inverse, top_k, score_before)
    return dx, (ds if score_before else None), None, None, None, None, None


dispatch.register_autograd(_dispatch_bwd, setup_context=_dispatch_setup)


# ---------------------------------------------------------------------------
# Experts: y = swiglu(clamp(routed @ w13[e]^T)) @ w2[e]^T (npu_gmm.py:21-40)
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::experts", mutates_args=())
def experts(routed: Tensor, w13: Tensor, w2: Tensor, offs: Tensor, swiglu_limit: Optional[float],
            keep_activations: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(y [M, D], h [M, 2H], a [M, H], w13_bf16, w2_bf16).  h and a (the saved
    pre-activation and SwiGLU output for the backward) are empty unless
    keep_activations.  Weights that are not bf16 (the reference's fp32
    nn.Parameters, npu_gmm.py:63-64, cast per call at :31 and :38) are cast
    once here; with keep_activations the bf16 copies are returned too, so
    the backward's GEMMs reuse them instead of casting again (empty for bf16
    weights, which the backward reads directly)."""
    w13b, w2b = _bf(w13), _bf(w2)
    a, h = ops.grouped_mm_swiglu(routed, w13b, offs, swiglu_limit, save_h=keep_activations)
    y = ops.grouped_mm_unpermute(a, w2b, offs)
    if not keep_activations:
        return y, _empty(routed), _empty(routed), _empty(routed), _empty(routed)
    return (y, h, a, w13b if w13.dtype != _BF16 else _empty(routed),
            w2b if w2.dtype != _BF16 else _empty(routed))


@experts.register_fake
def _(routed, w13, w2, offs, swiglu_limit, keep_activations):
    M, H, D = routed.shape[0], w13.shape[1] // 2, w2.shape[1]
    y = routed.new_empty((M, D), dtype=_BF16)
    e = lambda: routed.new_empty((0,))  # noqa: E731  (distinct tensors, as the real op returns)
    if not keep_activations:
        return y, e(), e(), e(), e()
    return (y, routed.new_empty((M, 2 * H), dtype=_BF16), routed.new_empty((M, H), dtype=_BF16),
            w13.new_empty(w13.shape, dtype=_BF16) if w13.dtype != _BF16 else e(),
            w2.new_empty(w2.shape, dtype=_BF16) if w2.dtype != _BF16 else e())


@torch.library.custom_op("ttamd::experts_backward", mutates_args=())
def experts_backward(dy: Tensor, routed: Tensor, h: Tensor, a: Tensor, w13: Tensor, w2: Tensor, offs: Tensor,
                     swiglu_limit: Optional[float], need_d_routed: bool, need_dw13: bool,
                     need_dw2: bool, w13_dtype: torch.dtype, w2_dtype: torch.dtype) -> tuple[Tensor, Tensor, Tensor]:
    """(d_routed bf16 [M, D], dw13 in w13_dtype, dw2 in w2_dtype); a gradient
    not asked for is an empty tensor.  w13 / w2 are the bf16 weights the
    forward used; gradients of weights that are not bf16 are accumulated and
    written in fp32 by the wgrad kernel."""
    dy = dy.to(_BF16).contiguous()
    w13b, w2b = _bf(w13), _bf(w2)
    E = w13.shape[0]
    dh, _ = ops.grouped_mm_dgrad_swiglu(dy, w2b, h, offs, swiglu_limit)
    dw2 = _empty(w2)
    dw13 = _empty(w13)
    d_routed = _empty(routed)
    if need_dw2:
        dw2 = ops.grouped_mm_wgrad(dy, a, offs, E, _F32 if w2_dtype != _BF16 else _BF16).to(w2_dtype)
    if need_dw13:
        dw13 = ops.grouped_mm_wgrad(dh, routed, offs, E, _F32 if w13_dtype != _BF16 else _BF16).to(w13_dtype)
    if need_d_routed:
        d_routed = ops.grouped_mm_dgrad(dh, w13b, offs)
    return d_routed, dw13, dw2


@experts_backward.register_fake
def _(dy, routed, h, a, w13, w2, offs, swiglu_limit, need_d_routed, need_dw13, need_dw2, w13_dtype, w2_dtype):
    return (routed.new_empty(routed.shape if need_d_routed else (0,), dtype=_BF16),
            w13.new_empty(w13.shape if need_dw13 else (0,), dtype=w13_dtype),
            w2.new_empty(w2.shape if need_dw2 else (0,), dtype=w2_dtype))


def _experts_setup(ctx, inputs, output):
    routed, w13, w2, offs, limit, keep = inputs
    _, h, a, w13b, w2b = output
    # the backward's GEMMs read the forward's bf16 weights: its cast copies
    # for fp32 (or other) weights, the parameters themselves when bf16
    ctx.save_for_backward(routed, h, a, w13b if w13b.numel() else w13, w2b if w2b.numel() else w2, offs)
    ctx.limit = limit
    ctx.keep = keep
    ctx.wdtypes = (w13.dtype, w2.dtype)
    # h, a and the weight copies are outputs for the backward only: autograd
    # must not fill zero gradients for them
    ctx.set_materialize_grads(False)


def _experts_bwd(ctx, dy, _dh, _da, _dw13b, _dw2b):
    if dy is None:
        return None, None, None, None, None, None
    routed, h, a, w13, w2, offs = ctx.saved_tensors
    if not ctx.keep:
        raise RuntimeError("ttamd::experts ran without keep_activations=True; its backward needs h and a")
    need = ctx.needs_input_grad
    d_routed, dw13, dw2 = experts_backward(dy, routed, h, a, w13, w2, offs, ctx.limit, need[0], need[1], need[2],
                                           ctx.wdtypes[0], ctx.wdtypes[1])
    return (d_routed if need[0] else None, dw13 if need[1] else None, dw2 if need[2] else None, None, None, None)


experts.register_autograd(_experts_bwd, setup_context=_experts_setup)


# ---------------------------------------------------------------------------
# Combine: out[t] = sum_k w(t,k) y[pos(t,k)] (w = score after the experts, else 1)
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::combine", mutates_args=())
def combine(y: Tensor, scores_flat: Tensor, sorted_indices: Tensor, inverse: Tensor, top_k: int,
            score_after: bool) -> Tensor:
    return ops.combine(y, inverse, scores_flat if score_after else None, top_k)


@combine.register_fake
def _(y, scores_flat, sorted_indices, inverse, top_k, score_after):
    return y.new_empty((y.shape[0] // top_k, y.shape[1]))


@torch.library.custom_op("ttamd::combine_backward", mutates_args=())
def combine_backward(dout: Tensor, y: Tensor, scores_flat: Tensor, sorted_indices: Tensor, top_k: int,
                     score_after: bool, need_dscores: bool) -> tuple[Tensor, Tensor]:
    """(dy [M, D], d scores_flat [M] (empty unless asked for))."""
    need_ds = score_after and need_dscores
    dy, ds = ops.token_unpermute_grad(dout.to(_BF16).contiguous(), sorted_indices,
                                      scores_flat if score_after else None, y if need_ds else None, top_k,
                                      need_probs_grad=need_ds)
    return dy, (ds if need_ds else _empty(scores_flat))


@combine_backward.register_fake
def _(dout, y, scores_flat, sorted_indices, top_k, score_after, need_dscores):
    return y.new_empty(y.shape), scores_flat.new_empty(scores_flat.shape if (score_after and need_dscores) else (0,))


def _combine_setup(ctx, inputs, output):
    y, scores_flat, sorted_indices, _inv, top_k, score_after = inputs
    ctx.save_for_backward(y, scores_flat, sorted_indices)
    ctx.cfg = (top_k, score_after)


def _combine_bwd(ctx, dout):
    y, scores_flat, sorted_indices = ctx.saved_tensors
    top_k, score_after = ctx.cfg
    need_ds = score_after and ctx.needs_input_grad[1]
    dy, ds = combine_backward(dout, y, scores_flat, sorted_indices, top_k, score_after, need_ds)
    return dy, (ds if need_ds else None), None, None, None, None


combine.register_autograd(_combine_bwd, setup_context=_combine_setup)


# ---------------------------------------------------------------------------
# Inference-only fused stages (no gradient)
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::moe_experts_forward", mutates_args=())
def moe_experts_forward(x: Tensor, sorted_indices: Tensor, offsets: Tensor, sorted_scores: Tensor, w13: Tensor,
                        w2: Tensor, top_k: int, score_before: bool, swiglu_limit: Optional[float]) -> Tensor:
    """ttamd_moe_experts_forward: dispatch -> w13 + SwiGLU -> w2 + score ->
    combine in one C-ABI call; offsets are route's exclusive [E + 1]."""
    r = ops.RouteResult(None, offsets, sorted_indices, None, sorted_scores)
    return ops.experts_forward(x, r, _bf(w13), _bf(w2), top_k, score_before, swiglu_limit)


@moe_experts_forward.register_fake
def _(x, sorted_indices, offsets, sorted_scores, w13, w2, top_k, score_before, swiglu_limit):
    return x.new_empty(x.shape, dtype=_BF16)


@torch.library.custom_op("ttamd::shared_expert_add", mutates_args=())
def shared_expert_add(routed_out: Tensor, x: Tensor, w13_shared: Tensor, w2_shared: Tensor,
                      gate_logits: Optional[Tensor], swiglu_limit: Optional[float]) -> Tensor:
    """routed_out + g * shared_expert(x) as a new tensor (ttamd_shared_expert_add)."""
    out = routed_out.to(_BF16).contiguous().clone()
    ops.shared_expert_add(out, x.to(_BF16), _bf(w13_shared), _bf(w2_shared),
                          None if gate_logits is None else gate_logits.float(), swiglu_limit)
    return out


@shared_expert_add.register_fake
def _(routed_out, x, w13_shared, w2_shared, gate_logits, swiglu_limit):
    return routed_out.new_empty(routed_out.shape, dtype=_BF16)


# ---------------------------------------------------------------------------
# Row permute / unpermute of the dispatcher (npu_permute.py:63-88): rows move
# bit for bit in their own dtype; each op's backward is the other
# ---------------------------------------------------------------------------
@torch.library.custom_op("ttamd::token_permute", mutates_args=())
def token_permute(rows: Tensor, labels: Tensor, num_labels: int) -> tuple[Tensor, Tensor]:
    """(permuted rows [M, D], sorted_indices int32 [M]) with permuted[j] =
    rows[sorted_indices[j]], sorted_indices the stable order of the labels."""
    r = ops.route(labels, num_labels)
    return ops.gather_rows_exact(rows, r.sorted_indices), r.sorted_indices


@token_permute.register_fake
def _(rows, labels, num_labels):
    return rows.new_empty(rows.shape), labels.new_empty((labels.numel(),), dtype=_I32)


@torch.library.custom_op("ttamd::token_unpermute", mutates_args=())
def token_unpermute(permuted: Tensor, sorted_indices: Tensor) -> Tensor:
    """out[sorted_indices[j]] = permuted[j]."""
    return ops.scatter_rows_exact(permuted.contiguous(), sorted_indices.to(_I32))


@token_unpermute.register_fake
def _(permuted, sorted_indices):
    return permuted.new_empty(permuted.shape)


@torch.library.custom_op("ttamd::token_gather", mutates_args=())
def token_gather(rows: Tensor, sorted_indices: Tensor) -> Tensor:
    """out[j] = rows[sorted_indices[j]] (the backward of token_unpermute)."""
    return ops.gather_rows_exact(rows.contiguous(), sorted_indices.to(_I32))


@token_gather.register_fake
def _(rows, sorted_indices):
    return rows.new_empty((sorted_indices.numel(), rows.shape[1]))


def _permute_setup(ctx, inputs, output):
    ctx.save_for_backward(output[1])
    ctx.set_materialize_grads(False)


def _permute_bwd(ctx, g_permuted, _g_idx):
    if g_permuted is None:
        return None, None, None
    (sorted_indices,) = ctx.saved_tensors
    return token_unpermute(g_permuted, sorted_indices), None, None


token_permute.register_autograd(_permute_bwd, setup_context=_permute_setup)


def _unpermute_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])


def _unpermute_bwd(ctx, g_out):
    (sorted_indices,) = ctx.saved_tensors
    return token_gather(g_out, sorted_indices), None


token_unpermute.register_autograd(_unpermute_bwd, setup_context=_unpermute_setup)


def _gather_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])


def _gather_bwd(ctx, g_out):
    (sorted_indices,) = ctx.saved_tensors
    return token_unpermute(g_out, sorted_indices), None


token_gather.register_autograd(_gather_bwd, setup_context=_gather_setup)
