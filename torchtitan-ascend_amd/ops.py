"""Torch-facing functional ops of the MoE expert path.

Every op allocates its outputs with torch's caching allocator, then calls the
C ABI of libttamd_moe.so on torch's current HIP stream.  There is no CPU or
eager-torch fallback: tensors must live on a HIP device and the library must
be built, otherwise the op raises.

Conventions (shared with include/ttamd_moe.h):
  * bf16 activations/weights, fp32 routing scores, int32 index maps;
  * flat slot s = t * top_k + k (the order of selected_experts_indices.view(-1));
  * `offs` = inclusive cumsum of per-expert row counts, int32 [E]
    (torchtitanturbo/models/common/npu_gmm.py:29).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib

_BF16 = torch.bfloat16


def _p(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _gpu(name: str, t: torch.Tensor) -> torch.device:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; the MoE expert path runs only on a HIP device (no CPU fallback)"
        )
    return t.device


def _same_device(dev: torch.device, **tensors) -> None:
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise RuntimeError(f"{name} is on {t.device}, expected {dev}")


def _want(name: str, t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    return t.contiguous()


def _ws(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=dev)


def _limit(swiglu_limit: float | None) -> float:
    if swiglu_limit is None:
        return math.nan
    if swiglu_limit < 0:
        raise ValueError(f"swiglu_limit must be >= 0 or None, got {swiglu_limit}")
    return float(swiglu_limit)


# ---------------------------------------------------------------------------
# Routing
# ---------------------------------------------------------------------------
@dataclass
class RouteResult:
    """Output of `route`: histogram, group offsets and the stable order."""

    counts: torch.Tensor  # int32 [E]
    offsets: torch.Tensor  # int32 [E+1], exclusive (offsets[0] = 0)
    sorted_indices: torch.Tensor  # int32 [M]: j-th flat slot in stable expert order
    inverse: torch.Tensor  # int32 [M]: position of flat slot s
    sorted_scores: torch.Tensor | None  # fp32 [M] or None
    # uint8 tile table of the expert-sorted rows for the forward grouped
    # GEMMs (router_route builds it; experts_forward reuses it)
    plan: torch.Tensor | None = None

    @property
    def offs(self) -> torch.Tensor:
        """Inclusive offsets int32 [E] in torch._grouped_mm's convention."""
        return self.offsets[1:]


def router_topk(
    logits: torch.Tensor,
    top_k: int,
    score_func: str = "softmax",
    route_norm: bool = False,
    route_scale: float = 1.0,
    expert_bias: torch.Tensor | None = None,
    norm_eps: float = 1e-20,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k selection of the router (upstream TokenChoiceTopKRouter; in-reference
    closed form torchtitanturbo/models/qwen3_5/model.py:757-765).

    Returns (top_scores fp32 [T, K], selected_experts_indices int64 [T, K]),
    sorted by descending score, ties broken towards the lower expert id.
    """
    dev = _gpu("logits", logits)
    if logits.dim() != 2:
        raise ValueError("logits must be [T, E]")
    logits = logits.float().contiguous()
    T, E = logits.shape
    funcs = {"softmax": 0, "sigmoid": 1}
    if score_func not in funcs:
        raise ValueError(f"score_func must be one of {sorted(funcs)}")
    if expert_bias is not None:
        _same_device(dev, expert_bias=expert_bias)
        expert_bias = expert_bias.float().contiguous()
        if expert_bias.shape != (E,):
            raise ValueError("expert_bias must be [E]")
    scores = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    _lib.call(
        "ttamd_router_topk", _p(logits), _p(expert_bias), T, E, top_k, funcs[score_func],
        int(bool(route_norm)), float(norm_eps), float(route_scale), _p(scores), _p(idx), _stream(dev),
    )
    return scores, idx


def router_fused(
    x: torch.Tensor,
    w_router: torch.Tensor,
    top_k: int,
    score_func: str = "softmax",
    route_norm: bool = False,
    route_scale: float = 1.0,
    expert_bias: torch.Tensor | None = None,
    norm_eps: float = 1e-20,
    return_logits: bool = False,
):
    """Gate GEMM + score + top-k in one kernel (upstream TokenChoiceTopKRouter;
    in-reference closed form torchtitanturbo/models/qwen3_5/model.py:752-766).

    x bf16 [T, D] (any leading shape), w_router bf16 [E, D].  The logits are
    the bf16 F.linear output; selection as `router_topk` on them.  Returns
    (top_scores fp32 [T, K], selected_experts_indices int64 [T, K]) and, with
    return_logits, the bf16 logits [T, E] as a third element.
    """
    dev = _gpu("x", x)
    x = _want("x", x.reshape(-1, x.shape[-1]), _BF16)
    w_router = _want("w_router", w_router, _BF16)
    T, D = x.shape
    E, D2 = w_router.shape
    if D2 != D:
        raise ValueError(f"w_router must be [E, {D}], got {tuple(w_router.shape)}")
    funcs = {"softmax": 0, "sigmoid": 1}
    if score_func not in funcs:
        raise ValueError(f"score_func must be one of {sorted(funcs)}")
    if expert_bias is not None:
        _same_device(dev, expert_bias=expert_bias)
        expert_bias = expert_bias.float().contiguous()
        if expert_bias.shape != (E,):
            raise ValueError("expert_bias must be [E]")
    scores = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    logits = torch.empty(T, E, dtype=_BF16, device=dev) if return_logits else None
    ws = _ws(_lib.load().ttamd_router_workspace_bytes(T, E, D), dev)
    _lib.call(
        "ttamd_router_fused", _p(x), _p(w_router), _p(expert_bias), T, E, D, top_k, funcs[score_func],
        int(bool(route_norm)), float(norm_eps), float(route_scale), _p(scores), _p(idx), _p(logits), _p(ws),
        ws.numel(), _stream(dev),
    )
    if return_logits:
        return scores, idx, logits
    return scores, idx


def router_backward(
    grad_top_scores: torch.Tensor,
    top_indices: torch.Tensor,
    logits: torch.Tensor,
    x: torch.Tensor,
    w_router: torch.Tensor,
    score_func: str = "softmax",
    route_norm: bool = False,
    route_scale: float = 1.0,
    norm_eps: float = 1e-20,
    need_dx: bool = True,
    need_dw: bool = True,
    dw_dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Backward of the router forward (ttamd_router_backward): from
    d(top_scores) [T, K], the picks and the forward's bf16 logits [T, E] to
    dx bf16 [T, D] and dW_r [E, D] (fp32 or bf16)."""
    dev = _gpu("grad_top_scores", grad_top_scores)
    x = _want("x", x.reshape(-1, x.shape[-1]), _BF16)
    w_router = _want("w_router", w_router, _BF16)
    logits = _want("logits", logits, _BF16)
    T, D = x.shape
    E = w_router.shape[0]
    K = top_indices.shape[-1]
    g = grad_top_scores.reshape(T, K).float().contiguous()
    idx = top_indices.reshape(T, K).to(torch.int64).contiguous()
    if tuple(logits.shape) != (T, E):
        raise ValueError(f"logits must be [{T}, {E}], got {tuple(logits.shape)}")
    if dw_dtype not in (torch.float32, _BF16):
        raise TypeError("dw_dtype must be float32 or bfloat16")
    funcs = {"softmax": 0, "sigmoid": 1}
    dx = torch.empty(T, D, dtype=_BF16, device=dev) if need_dx else None
    dw = torch.empty(E, D, dtype=dw_dtype, device=dev) if need_dw else None
    ws = _ws(_lib.load().ttamd_router_backward_workspace_bytes(T, E, D), dev)
    _lib.call(
        "ttamd_router_backward", _p(g), _p(idx), _p(logits), _p(x), _p(w_router), T, E, D, K, funcs[score_func],
        int(bool(route_norm)), float(norm_eps), float(route_scale), _p(dx), _p(dw), int(dw_dtype == torch.float32),
        _p(ws), ws.numel(), _stream(dev),
    )
    return dx, dw


def router_route(
    x: torch.Tensor,
    w_router: torch.Tensor,
    top_k: int,
    score_func: str = "softmax",
    route_norm: bool = False,
    route_scale: float = 1.0,
    expert_bias: torch.Tensor | None = None,
    norm_eps: float = 1e-20,
    tokens_per_expert: torch.Tensor | None = None,
    with_inverse: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, RouteResult]:
    """Router forward + dispatch order in one C-ABI call (ttamd_router_route):
    the picks of `router_fused`, then the histogram and stable order of
    `route` over them, plus the grouped GEMMs' tile table (RouteResult.plan).
    tokens_per_expert (fp32 [E], optional) is incremented by the counts, as
    upstream's router.tokens_per_expert buffer is.  Returns (top_scores
    fp32 [T, K], selected_experts_indices int64 [T, K], RouteResult with
    sorted_scores = top_scores.view(-1)[sorted_indices])."""
    dev = _gpu("x", x)
    if torch.is_grad_enabled() and (x.requires_grad or w_router.requires_grad):
        raise RuntimeError(
            "router_route is the inference path (its scores carry no autograd); for training use "
            "functional.router (differentiable) followed by route"
        )
    x = _want("x", x.reshape(-1, x.shape[-1]), _BF16)
    w_router = _want("w_router", w_router, _BF16)
    T, D = x.shape
    E, D2 = w_router.shape
    if D2 != D:
        raise ValueError(f"w_router must be [E, {D}], got {tuple(w_router.shape)}")
    funcs = {"softmax": 0, "sigmoid": 1}
    if score_func not in funcs:
        raise ValueError(f"score_func must be one of {sorted(funcs)}")
    if expert_bias is not None:
        _same_device(dev, expert_bias=expert_bias)
        expert_bias = expert_bias.float().contiguous()
        if expert_bias.shape != (E,):
            raise ValueError("expert_bias must be [E]")
    if tokens_per_expert is not None:
        _same_device(dev, tokens_per_expert=tokens_per_expert)
        if tokens_per_expert.dtype != torch.float32 or tokens_per_expert.shape != (E,) or \
                not tokens_per_expert.is_contiguous():
            raise ValueError("tokens_per_expert must be a contiguous fp32 [E] tensor (updated in place)")
    M = T * top_k
    lib = _lib.load()
    scores = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    sorted_idx = torch.empty(M, dtype=torch.int32, device=dev)
    inverse = torch.empty(M, dtype=torch.int32, device=dev) if with_inverse else None
    sorted_scores = torch.empty(M, dtype=torch.float32, device=dev)
    plan = _ws(lib.ttamd_gemm_plan_bytes(M, E), dev)
    ws = _ws(lib.ttamd_router_route_workspace_bytes(T, E, D, top_k), dev)
    _lib.call(
        "ttamd_router_route", _p(x), _p(w_router), _p(expert_bias), T, E, D, top_k, funcs[score_func],
        int(bool(route_norm)), float(norm_eps), float(route_scale), _p(scores), _p(idx), _p(counts), _p(offsets),
        _p(sorted_idx), _p(inverse), _p(sorted_scores), _p(tokens_per_expert), _p(plan), plan.numel(), _p(ws),
        ws.numel(), _stream(dev),
    )
    return scores, idx, RouteResult(counts, offsets, sorted_idx, inverse, sorted_scores, plan)


def experts_forward(
    x: torch.Tensor,
    r: RouteResult,
    w13: torch.Tensor,
    w2: torch.Tensor,
    top_k: int,
    score_before_experts: bool,
    swiglu_limit: float | None = None,
) -> torch.Tensor:
    """The expert stage of the inference forward in one C-ABI call
    (ttamd_moe_experts_forward): dispatch -> w13 + SwiGLU -> w2 + score ->
    combine (npu_gmm.py:100-110 with :21-40) on the routing `r` (from
    `route` or `router_route`; r.sorted_scores must be set).  Both grouped
    GEMMs use r.plan when present.  x bf16 [T, D] -> out bf16 [T, D]."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    w13 = _want("w13", w13, _BF16)
    w2 = _want("w2", w2, _BF16)
    T, D = x.shape
    E, H2, D2 = w13.shape
    if D2 != D or H2 % 2 or tuple(w2.shape) != (E, D, H2 // 2):
        raise ValueError(f"w13 must be [E, 2H, {D}] and w2 [E, {D}, H]; got {tuple(w13.shape)}, {tuple(w2.shape)}")
    H = H2 // 2
    if r.sorted_scores is None:
        raise ValueError("experts_forward needs the routing scores (route(..., scores))")
    if r.sorted_indices.numel() != T * top_k:
        raise ValueError("routing does not match T * top_k rows")
    lib = _lib.load()
    out = torch.empty(T, D, dtype=_BF16, device=dev)
    ws = _ws(lib.ttamd_moe_experts_forward_workspace_bytes(T, D, H, E, top_k, int(bool(score_before_experts))), dev)
    plan = r.plan
    _lib.call(
        "ttamd_moe_experts_forward", _p(x), T, D, H, E, top_k, _p(r.sorted_indices), _p(r.offs.contiguous()),
        _p(r.sorted_scores), int(bool(score_before_experts)), _limit(swiglu_limit), _p(w13), _p(w2), _p(out),
        _p(plan), 0 if plan is None else plan.numel(), _p(ws), ws.numel(), _stream(dev),
    )
    return out


def route(
    selected_experts_indices: torch.Tensor,
    num_experts: int,
    scores: torch.Tensor | None = None,
) -> RouteResult:
    """Histogram + stable counting sort of the flat expert labels.

    Bit-exact equivalent of upstream dispatch's
    `histc(idx.view(-1), bins=E)` and `argsort(idx.view(-1), stable=True)`
    (reached from torchtitanturbo/models/common/npu_gmm.py:106-108).
    """
    dev = _gpu("selected_experts_indices", selected_experts_indices)
    labels = selected_experts_indices.reshape(-1)
    if labels.dtype not in (torch.int64, torch.int32):
        raise TypeError("expert indices must be int64 or int32")
    labels = labels.contiguous()
    M = labels.numel()
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_idx = torch.empty(M, dtype=torch.int32, device=dev)
    inverse = torch.empty(M, dtype=torch.int32, device=dev)
    sorted_scores = None
    sc = None
    if scores is not None:
        _same_device(dev, scores=scores)
        sc = scores.reshape(-1).float().contiguous()
        if sc.numel() != M:
            raise ValueError("scores must have one entry per expert choice")
        sorted_scores = torch.empty(M, dtype=torch.float32, device=dev)
    lib = _lib.load()
    wsb = lib.ttamd_route_workspace_bytes(M, num_experts)
    ws = _ws(wsb, dev)
    _lib.call(
        "ttamd_moe_route", _p(labels), int(labels.dtype == torch.int64), M, num_experts, _p(sc),
        _p(counts), _p(offsets), _p(sorted_idx), _p(inverse), _p(sorted_scores), _p(ws), ws.numel(),
        _stream(dev),
    )
    return RouteResult(counts, offsets, sorted_idx, inverse, sorted_scores)


def gather_rows(
    x: torch.Tensor, src_index: torch.Tensor, top_k: int = 1, row_scale: torch.Tensor | None = None
) -> torch.Tensor:
    """out[j] = x[src_index[j] // top_k] (* row_scale[j] in fp32, rounded once)."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    src_index = _want("src_index", src_index, torch.int32)
    _same_device(dev, src_index=src_index, row_scale=row_scale)
    rows = src_index.numel()
    D = x.shape[-1]
    out = torch.empty(rows, D, dtype=_BF16, device=dev)
    if row_scale is not None:
        row_scale = _want("row_scale", row_scale, torch.float32)
    _lib.call(
        "ttamd_moe_gather_rows", _p(x), _p(src_index), _p(row_scale), x.numel() // D, rows, D, top_k,
        _p(out), _stream(dev),
    )
    return out


def permute_rows(
    x: torch.Tensor, r: "RouteResult", top_k: int, scores_flat: torch.Tensor | None = None
) -> torch.Tensor:
    """The dispatcher's row permute for a route() result: routed[j] =
    x[sorted_indices[j] // K] (* score).  top_k > 1 uses the scatter form
    (each token row read once, K writes); top_k == 1 the gather form
    (sequential writes), whichever moves fewer HBM bytes."""
    if top_k == 1:
        return gather_rows(x, r.sorted_indices, 1, r.sorted_scores if scores_flat is not None else None)
    return dispatch_rows(x, r.inverse, top_k, scores_flat)


def dispatch_rows(
    x: torch.Tensor, inverse: torch.Tensor, top_k: int, scores_flat: torch.Tensor | None = None
) -> torch.Tensor:
    """out[inverse[t*K + k]] = x[t] (* scores_flat[t*K + k], rounded once): the
    permute rows of gather_rows(x, sorted_indices, K, sorted_scores), with
    each token row read once."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    inverse = _want("inverse", inverse, torch.int32)
    _same_device(dev, inverse=inverse, scores_flat=scores_flat)
    T, D = x.shape
    if inverse.numel() != T * top_k:
        raise ValueError(f"inverse has {inverse.numel()} entries, expected {T * top_k}")
    if scores_flat is not None:
        scores_flat = _want("scores_flat", scores_flat, torch.float32)
    out = torch.empty(T * top_k, D, dtype=_BF16, device=dev)
    _lib.call("ttamd_moe_dispatch_rows", _p(x), _p(inverse), _p(scores_flat), T, D, top_k, _p(out), _stream(dev))
    return out


def _rows_as_bf16(name: str, t: torch.Tensor) -> torch.Tensor:
    """A contiguous 2-D tensor of 2- or 4-byte elements viewed as bf16 bit
    pairs [rows, cols * elsize / 2]: the row movers copy 16-byte chunks
    unchanged when no scale is applied, so rows of any such dtype move bit
    for bit."""
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.element_size() not in (2, 4) or t.dtype.is_complex:
        raise TypeError(f"{name}: rows of {t.dtype} cannot be moved (2- or 4-byte elements only)")
    return t.contiguous().view(_BF16)


def gather_rows_exact(x: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """out[j] = x[index[j]], bit for bit, for bf16 / fp16 / fp32 rows."""
    dev = _gpu("x", x)
    index = _want("index", index, torch.int32)
    _same_device(dev, index=index)
    xv = _rows_as_bf16("x", x)
    rows, W = index.numel(), xv.shape[1]
    out = torch.empty(rows, W, dtype=_BF16, device=dev)
    if W % 8:
        raise ValueError(f"row width of {x.shape[1]} {x.dtype} elements is not a multiple of 16 bytes")
    _lib.call("ttamd_moe_gather_rows", _p(xv), _p(index), None, xv.shape[0], rows, W, 1, _p(out), _stream(dev))
    return out.view(x.dtype)


def scatter_rows_exact(x: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """out[index[j]] = x[j], bit for bit (index a permutation of the rows)."""
    dev = _gpu("x", x)
    index = _want("index", index, torch.int32)
    _same_device(dev, index=index)
    xv = _rows_as_bf16("x", x)
    if index.numel() != xv.shape[0]:
        raise ValueError(f"index has {index.numel()} entries for {xv.shape[0]} rows")
    T, W = xv.shape
    if W % 8:
        raise ValueError(f"row width of {x.shape[1]} {x.dtype} elements is not a multiple of 16 bytes")
    out = torch.empty(T, W, dtype=_BF16, device=dev)
    _lib.call("ttamd_moe_dispatch_rows", _p(xv), _p(index), None, T, W, 1, _p(out), _stream(dev))
    return out.view(x.dtype)


def token_permute(
    tokens: torch.Tensor, indices: torch.Tensor, num_experts: int, return_counts: bool = False
):
    """Drop-in for torch_npu.npu_moe_token_permute(tokens, indices)
    (torchtitanturbo/models/common/npu_permute.py:74-76).

    indices [T] or [T, K] expert labels; returns (permuted [T*K, D],
    sorted_indices int32 [T*K]) with sorted_indices the stable argsort of the
    flat labels.  `num_experts` bounds the label range.
    """
    dev = _gpu("tokens", tokens)
    tokens = _want("tokens", tokens, _BF16)
    _same_device(dev, indices=indices)
    T, D = tokens.shape
    topk = 1 if indices.dim() == 1 else indices.shape[-1]
    labels = indices.reshape(-1).contiguous()
    if labels.dtype not in (torch.int64, torch.int32):
        raise TypeError("indices must be int64 or int32")
    if labels.numel() != T * topk:
        raise ValueError("indices must have T * top_k entries")
    M = T * topk
    permuted = torch.empty(M, D, dtype=_BF16, device=dev)
    sorted_idx = torch.empty(M, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws = _ws(lib.ttamd_route_workspace_bytes(M, num_experts), dev)
    _lib.call(
        "ttamd_moe_token_permute", _p(tokens), _p(labels), int(labels.dtype == torch.int64), T, D, topk,
        num_experts, _p(permuted), _p(sorted_idx), _p(counts), _p(ws), ws.numel(), _stream(dev),
    )
    if return_counts:
        return permuted, sorted_idx, counts
    return permuted, sorted_idx


def token_unpermute(
    permuted: torch.Tensor,
    sorted_indices: torch.Tensor,
    probs: torch.Tensor | None = None,
    top_k: int = 1,
) -> torch.Tensor:
    """Drop-in for torch_npu._npu_moe_token_unpermute_with_routing_map
    (npu_permute.py:23-30): out[t] = sum_k probs[t,k] * permuted[j(t,k)]."""
    dev = _gpu("permuted", permuted)
    permuted = _want("permuted", permuted, _BF16)
    sorted_indices = _want("sorted_indices", sorted_indices, torch.int32)
    _same_device(dev, sorted_indices=sorted_indices, probs=probs)
    M, D = permuted.shape
    if M % top_k:
        raise ValueError("permuted rows must be a multiple of top_k")
    T = M // top_k
    if probs is not None:
        probs = probs.reshape(-1).float().contiguous()
    out = torch.empty(T, D, dtype=_BF16, device=dev)
    lib = _lib.load()
    ws = _ws(lib.ttamd_unpermute_workspace_bytes(T, top_k), dev)
    _lib.call(
        "ttamd_moe_token_unpermute", _p(permuted), _p(sorted_indices), _p(probs), T, D, top_k, _p(out),
        _p(ws), ws.numel(), _stream(dev),
    )
    return out


def token_unpermute_grad(
    grad_out: torch.Tensor,
    sorted_indices: torch.Tensor,
    probs: torch.Tensor | None = None,
    permuted: torch.Tensor | None = None,
    top_k: int = 1,
    need_probs_grad: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Drop-in for torch_npu.npu_moe_token_unpermute_with_routing_map_grad
    (npu_permute.py:41-50).  Returns (grad_permuted, grad_probs or None)."""
    dev = _gpu("grad_out", grad_out)
    grad_out = _want("grad_out", grad_out, _BF16)
    sorted_indices = _want("sorted_indices", sorted_indices, torch.int32)
    T, D = grad_out.shape
    M = T * top_k
    if probs is not None:
        probs = probs.reshape(-1).float().contiguous()
    gp = None
    if need_probs_grad:
        if probs is None or permuted is None:
            raise ValueError("probs gradient needs probs and permuted")
        permuted = _want("permuted", permuted, _BF16)
        gp = torch.empty(M, dtype=torch.float32, device=dev)
    g = torch.empty(M, D, dtype=_BF16, device=dev)
    _lib.call(
        "ttamd_moe_token_unpermute_grad", _p(grad_out), _p(sorted_indices), _p(probs),
        _p(permuted if need_probs_grad else None), T, D, top_k, _p(g), _p(gp), _stream(dev),
    )
    return g, gp


def combine(
    permuted: torch.Tensor, inverse: torch.Tensor, probs: torch.Tensor | None, top_k: int
) -> torch.Tensor:
    """out[t] = sum_k probs[t,k] * permuted[inverse[t*K+k]] (fp32 accumulate)."""
    dev = _gpu("permuted", permuted)
    permuted = _want("permuted", permuted, _BF16)
    inverse = _want("inverse", inverse, torch.int32)
    M, D = permuted.shape
    T = M // top_k
    if probs is not None:
        probs = probs.reshape(-1).float().contiguous()
    out = torch.empty(T, D, dtype=_BF16, device=dev)
    _lib.call("ttamd_moe_combine", _p(permuted), _p(inverse), _p(probs), T, D, top_k, _p(out), _stream(dev))
    return out


def rowdot_scatter(a: torch.Tensor, b: torch.Tensor, index: torch.Tensor, div: int) -> torch.Tensor:
    """out[index[j]] = <a[j], b[index[j] // div]> in fp32 (a and out have the same rows)."""
    dev = _gpu("a", a)
    a = _want("a", a, _BF16)
    b = _want("b", b, _BF16)
    index = _want("index", index, torch.int32)
    out = torch.empty(a.shape[0], dtype=torch.float32, device=dev)
    _lib.call(
        "ttamd_moe_rowdot", _p(a), _p(b), _p(index), div, 1, a.shape[0], b.shape[0], a.shape[1], _p(out),
        _stream(dev),
    )
    return out


def sum_topk(y: torch.Tensor, top_k: int) -> torch.Tensor:
    dev = _gpu("y", y)
    y = _want("y", y, _BF16)
    M, D = y.shape
    out = torch.empty(M // top_k, D, dtype=_BF16, device=dev)
    _lib.call("ttamd_moe_sum_topk", _p(y), M // top_k, D, top_k, _p(out), _stream(dev))
    return out


def group_labels(counts_group: torch.Tensor, num_local_experts: int, num_rows: int) -> torch.Tensor:
    """Labels of rows grouped (rank, local expert): row in group g gets g % E_loc
    (torchtitanturbo/models/common/npu_permute.py:68-72), computed without a host sync."""
    dev = _gpu("counts_group", counts_group)
    cg = counts_group.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty(num_rows, dtype=torch.int32, device=dev)
    _lib.call("ttamd_moe_group_labels", _p(cg), cg.numel(), num_local_experts, num_rows, _p(out), _stream(dev))
    return out


# ---------------------------------------------------------------------------
# Grouped GEMMs
# ---------------------------------------------------------------------------
def _gemm_ws(M: int, E: int, dev: torch.device) -> torch.Tensor:
    return _ws(_lib.load().ttamd_gemm_workspace_bytes(M, E), dev)


def probe_next_gemm(start: "torch.cuda.Event | None", end: "torch.cuda.Event | None") -> None:
    """Arm the kernel timing probe (ttamd_probe_next_gemm): the next forward
    grouped-GEMM op (grouped_mm*, bf16 or fp8) records `start` and `end` on its
    stream immediately around its main kernel, excluding the tile-table
    kernel before it.  The events need enable_timing=True; they are recorded
    once here so that the HIP events exist.  None, None disarms."""
    if (start is None) != (end is None):
        raise ValueError("probe_next_gemm: give both events or neither")
    if start is None:
        _lib.call("ttamd_probe_next_gemm", None, None)
        return
    for e in (start, end):
        if not e.cuda_event:
            e.record()
    _lib.call("ttamd_probe_next_gemm", ctypes.c_void_p(start.cuda_event), ctypes.c_void_p(end.cuda_event))


def probe_launches(events: "list[torch.cuda.Event | None] | None") -> None:
    """Arm the launch-chain probe (ttamd_probe_launches) over the next
    len(events) // 2 kernel launches of the library's ops: launch i takes
    events[2 i] and events[2 i + 1] as its own start and end stamps, so
    events[2 i].elapsed_time(events[2 i + 1]) is launch i's kernel time, or
    runs unstamped when both are None.  The events need enable_timing=True
    (recorded once here so that the HIP events exist).  None (or an empty
    list) disarms."""
    if not events:
        _lib.call("ttamd_probe_launches", None, 0)
        return
    if len(events) % 2:
        raise ValueError("probe_launches: give an even number of events (start, end per launch)")
    for e in events:
        if e is not None and not e.cuda_event:
            e.record()
    arr = (ctypes.c_void_p * len(events))(*[None if e is None else e.cuda_event for e in events])
    _lib.call("ttamd_probe_launches", arr, len(events) // 2)


def _offs(offs: torch.Tensor, dev: torch.device) -> torch.Tensor:
    _same_device(dev, offs=offs)
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    return offs.contiguous()


def grouped_mm(x: torch.Tensor, w: torch.Tensor, offs: torch.Tensor) -> torch.Tensor:
    """out[m] = x[m] @ w[e(m)]^T, w [E, N, K]; torch._grouped_mm(x, w.transpose(-2, -1), offs)
    as called at torchtitanturbo/models/common/npu_gmm.py:17-18."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    w = _want("w", w, _BF16)
    offs = _offs(offs, dev)
    M, K = x.shape
    E, N, K2 = w.shape
    if K2 != K:
        raise ValueError(f"x has K={K}, w has K={K2}")
    out = torch.empty(M, N, dtype=_BF16, device=dev)
    ws = _gemm_ws(M, E, dev)
    _lib.call("ttamd_grouped_mm", _p(x), _p(w), _p(offs), M, E, N, K, _p(out), _p(ws), ws.numel(), _stream(dev))
    return out


def grouped_mm_swiglu(
    x: torch.Tensor, w13: torch.Tensor, offs: torch.Tensor, swiglu_limit: float | None = None, save_h: bool = False
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """a = swiglu(clamp(x @ w13[e]^T)) (npu_gmm.py:29-37); returns (a [M,H], h [M,2H] or None)."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    w13 = _want("w13", w13, _BF16)
    offs = _offs(offs, dev)
    M, D = x.shape
    E, H2, D2 = w13.shape
    if D2 != D or H2 % 2:
        raise ValueError(f"w13 must be [E, 2H, {D}], got {tuple(w13.shape)}")
    H = H2 // 2
    a = torch.empty(M, H, dtype=_BF16, device=dev)
    h = torch.empty(M, 2 * H, dtype=_BF16, device=dev) if save_h else None
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_swiglu", _p(x), _p(w13), _p(offs), M, E, H, D, _limit(swiglu_limit), _p(a), _p(h),
        _p(ws), ws.numel(), _stream(dev),
    )
    return a, h


def grouped_mm_swiglu_gather(
    tokens: torch.Tensor, src_index: torch.Tensor, src_div: int, w13: torch.Tensor, offs: torch.Tensor,
    swiglu_limit: float | None = None, save_h: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """grouped_mm_swiglu on the routed rows tokens[src_index[j] // src_div],
    gathered inside the GEMM's loads (no routed copy)."""
    dev = _gpu("tokens", tokens)
    tokens = _want("tokens", tokens, _BF16)
    src_index = _want("src_index", src_index, torch.int32)
    w13 = _want("w13", w13, _BF16)
    offs = _offs(offs, dev)
    T, D = tokens.shape
    M = src_index.numel()
    E, H2, D2 = w13.shape
    if D2 != D or H2 % 2:
        raise ValueError(f"w13 must be [E, 2H, {D}], got {tuple(w13.shape)}")
    H = H2 // 2
    a = torch.empty(M, H, dtype=_BF16, device=dev)
    h = torch.empty(M, 2 * H, dtype=_BF16, device=dev) if save_h else None
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_swiglu_gather", _p(tokens), T, _p(src_index), int(src_div), _p(w13), _p(offs), M, E, H,
        D, _limit(swiglu_limit), _p(a), _p(h), _p(ws), ws.numel(), _stream(dev),
    )
    return a, h


def grouped_mm_unpermute(
    a: torch.Tensor,
    w2: torch.Tensor,
    offs: torch.Tensor,
    row_scale: torch.Tensor | None = None,
    dest: torch.Tensor | None = None,
    num_dest_rows: int | None = None,
) -> torch.Tensor:
    """out[dest[j]] = row_scale[j] * (a[j] @ w2[e(j)]^T), w2 [E, D, H] (npu_gmm.py:38 + combine)."""
    dev = _gpu("a", a)
    a = _want("a", a, _BF16)
    w2 = _want("w2", w2, _BF16)
    offs = _offs(offs, dev)
    M, H = a.shape
    E, D, H2 = w2.shape
    if H2 != H:
        raise ValueError(f"w2 must be [E, D, {H}], got {tuple(w2.shape)}")
    if row_scale is not None:
        row_scale = _want("row_scale", row_scale, torch.float32)
    if dest is not None:
        dest = _want("dest", dest, torch.int32)
    nd = M if num_dest_rows is None else int(num_dest_rows)
    out = torch.empty(nd, D, dtype=_BF16, device=dev)
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_unpermute", _p(a), _p(w2), _p(offs), M, E, D, H, _p(row_scale), _p(dest), nd, _p(out),
        _p(ws), ws.numel(), _stream(dev),
    )
    return out


def grouped_mm_dgrad(dy: torch.Tensor, w: torch.Tensor, offs: torch.Tensor) -> torch.Tensor:
    """dx[m] = dy[m] @ w[e(m)], w [E, N, K] (backward of grouped_mm w.r.t. x)."""
    dev = _gpu("dy", dy)
    dy = _want("dy", dy, _BF16)
    w = _want("w", w, _BF16)
    offs = _offs(offs, dev)
    M, N = dy.shape
    E, N2, K = w.shape
    if N2 != N:
        raise ValueError("dy and w disagree on N")
    dx = torch.empty(M, K, dtype=_BF16, device=dev)
    ws = _gemm_ws(M, E, dev)
    _lib.call("ttamd_grouped_mm_dgrad", _p(dy), _p(w), _p(offs), M, E, N, K, _p(dx), _p(ws), ws.numel(), _stream(dev))
    return dx


def grouped_mm_dgrad_swiglu(
    dy: torch.Tensor, w2: torch.Tensor, h: torch.Tensor, offs: torch.Tensor,
    swiglu_limit: float | None = None, want_a: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """dh = swiglu_backward(dy @ w2[e], h); returns (dh [M, 2H], a [M, H] or None)."""
    dev = _gpu("dy", dy)
    dy = _want("dy", dy, _BF16)
    w2 = _want("w2", w2, _BF16)
    h = _want("h", h, _BF16)
    offs = _offs(offs, dev)
    M, D = dy.shape
    E, D2, H = w2.shape
    if D2 != D or h.shape != (M, 2 * H):
        raise ValueError("dy, w2 and h shapes disagree")
    dh = torch.empty(M, 2 * H, dtype=_BF16, device=dev)
    a = torch.empty(M, H, dtype=_BF16, device=dev) if want_a else None
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_dgrad_swiglu", _p(dy), _p(w2), _p(h), _p(offs), M, E, D, H, _limit(swiglu_limit),
        _p(dh), _p(a), _p(ws), ws.numel(), _stream(dev),
    )
    return dh, a


def grouped_mm_wgrad(
    dy: torch.Tensor, x: torch.Tensor, offs: torch.Tensor, num_experts: int, out_dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """dw[e] = dy_e^T @ x_e over each expert's rows; dw [E, N, K] in out_dtype (fp32 or bf16)."""
    dev = _gpu("dy", dy)
    dy = _want("dy", dy, _BF16)
    x = _want("x", x, _BF16)
    offs = _offs(offs, dev)
    M, N = dy.shape
    M2, K = x.shape
    if M2 != M:
        raise ValueError("dy and x must have the same rows")
    if out_dtype not in (torch.float32, _BF16):
        raise TypeError("wgrad output must be float32 or bfloat16")
    dw = torch.empty(num_experts, N, K, dtype=out_dtype, device=dev)
    ws = _gemm_ws(M, num_experts, dev)  # tail split of the leftover output tiles
    _lib.call(
        "ttamd_grouped_mm_wgrad", _p(dy), _p(x), _p(offs), M, num_experts, N, K, _p(dw),
        int(out_dtype == torch.float32), _p(ws), ws.numel(), _stream(dev),
    )
    return dw


# ---------------------------------------------------------------------------
# fp8 e4m3 experts (block scales, absmax / 448)
# ---------------------------------------------------------------------------
_U8 = torch.uint8


def shared_expert_add(
    out: torch.Tensor,
    x: torch.Tensor,
    w13_shared: torch.Tensor,
    w2_shared: torch.Tensor,
    gate_logits: torch.Tensor | None = None,
    swiglu_limit: float | None = None,
) -> torch.Tensor:
    """In place: out[t] += g(t) * FFN(x[t]) with FFN the shared SwiGLU expert
    (w13_shared [2H, D] gate-then-up, w2_shared [D, H]) and g = sigmoid(gate_logits)
    or 1 (torchtitanturbo/models/qwen3_5/model.py:796-809).  Returns out."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    w13_shared = _want("w13_shared", w13_shared, _BF16)
    w2_shared = _want("w2_shared", w2_shared, _BF16)
    if out.dtype != _BF16 or not out.is_contiguous():
        raise TypeError("out must be a contiguous bf16 tensor (it is updated in place)")
    T, D = x.shape
    H2, D2 = w13_shared.shape
    H = H2 // 2
    if D2 != D or H2 % 2 or tuple(w2_shared.shape) != (D, H) or tuple(out.shape) != (T, D):
        raise ValueError(f"shapes: x {tuple(x.shape)}, w13_shared {tuple(w13_shared.shape)}, "
                         f"w2_shared {tuple(w2_shared.shape)}, out {tuple(out.shape)}")
    _same_device(dev, out=out, w13_shared=w13_shared, w2_shared=w2_shared)
    if gate_logits is not None:
        gate_logits = _want("gate_logits", gate_logits.reshape(T), torch.float32)
    a = torch.empty(T, H, dtype=_BF16, device=dev)
    ws = _gemm_ws(T, 1, dev)
    _lib.call(
        "ttamd_shared_expert_add", _p(x), T, D, H, _p(w13_shared), _p(w2_shared), _p(gate_logits),
        _limit(swiglu_limit), _p(a), _p(out),
        _p(ws), ws.numel(), _stream(dev),
    )
    return out


def quantize_fp8_rows(
    x: torch.Tensor,
    src_index: torch.Tensor | None = None,
    src_div: int = 1,
    row_scale: torch.Tensor | None = None,
    num_rows: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row, per-128-channel e4m3 quantisation, optionally of gathered rows
    (row j = x[src_index[j] // src_div], times row_scale[j] rounded to bf16).
    Returns (q uint8 [R, K], scale_t fp32 [K / 128, R])."""
    dev = _gpu("x", x)
    x = _want("x", x, _BF16)
    n_in, K = x.shape
    if src_index is not None:
        src_index = _want("src_index", src_index, torch.int32)
        R = src_index.numel() if num_rows is None else int(num_rows)
    else:
        R = n_in if num_rows is None else int(num_rows)
    if row_scale is not None:
        row_scale = _want("row_scale", row_scale, torch.float32)
    q = torch.empty(R, K, dtype=_U8, device=dev)
    s = torch.empty(K // 128 if K % 128 == 0 else 0, R, dtype=torch.float32, device=dev)
    _lib.call(
        "ttamd_quantize_fp8_rows", _p(x), _p(src_index), int(src_div), _p(row_scale), n_in, R, K, _p(q), _p(s),
        _stream(dev),
    )
    return q, s


def quantize_fp8_blocks(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """128 x 128 block e4m3 quantisation of expert weights w [E, N, K].
    Returns (q uint8 [E, N, K], scale fp32 [E, N / 128, K / 128])."""
    dev = _gpu("w", w)
    w = _want("w", w, _BF16)
    E, N, K = w.shape
    q = torch.empty(E, N, K, dtype=_U8, device=dev)
    s = torch.empty(E, N // 128, K // 128, dtype=torch.float32, device=dev)
    _lib.call("ttamd_quantize_fp8_blocks", _p(w), E, N, K, _p(q), _p(s), _stream(dev))
    return q, s


def _fp8_operands(xq, sx_t, wq, sw, dev):
    xq = _want("xq", xq, _U8)
    sx_t = _want("sx_t", sx_t, torch.float32)
    wq = _want("wq", wq, _U8)
    sw = _want("sw", sw, torch.float32)
    M, K = xq.shape
    E, N, K2 = wq.shape
    if K2 != K:
        raise ValueError(f"xq has K={K}, wq has K={K2}")
    if sx_t.shape != (K // 128, M) or sw.shape != (E, N // 128, K // 128):
        raise ValueError("scale shapes do not match the operands")
    return xq, sx_t, wq, sw, M, K, E, N


def grouped_mm_fp8(xq: torch.Tensor, sx_t: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor,
                   offs: torch.Tensor) -> torch.Tensor:
    """fp8 grouped GEMM on dequantised operands, bf16 out [M, N]."""
    dev = _gpu("xq", xq)
    xq, sx_t, wq, sw, M, K, E, N = _fp8_operands(xq, sx_t, wq, sw, dev)
    offs = _offs(offs, dev)
    out = torch.empty(M, N, dtype=_BF16, device=dev)
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_fp8", _p(xq), _p(sx_t), _p(wq), _p(sw), _p(offs), M, E, N, K, _p(out), _p(ws),
        ws.numel(), _stream(dev),
    )
    return out


def grouped_mm_fp8_swiglu(
    xq: torch.Tensor, sx_t: torch.Tensor, w13q: torch.Tensor, s13: torch.Tensor, offs: torch.Tensor,
    swiglu_limit: float | None = None, save_h: bool = False,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """fp8 w13 GEMM + clamp + SwiGLU; returns (a [M, H] bf16, h [M, 2H] bf16 or None)."""
    dev = _gpu("xq", xq)
    xq, sx_t, w13q, s13, M, D, E, H2 = _fp8_operands(xq, sx_t, w13q, s13, dev)
    offs = _offs(offs, dev)
    H = H2 // 2
    a = torch.empty(M, H, dtype=_BF16, device=dev)
    h = torch.empty(M, 2 * H, dtype=_BF16, device=dev) if save_h else None
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_fp8_swiglu", _p(xq), _p(sx_t), _p(w13q), _p(s13), _p(offs), M, E, H, D,
        _limit(swiglu_limit), _p(a), _p(h), _p(ws), ws.numel(), _stream(dev),
    )
    return a, h


def grouped_mm_fp8_unpermute(
    aq: torch.Tensor, sa_t: torch.Tensor, w2q: torch.Tensor, s2: torch.Tensor, offs: torch.Tensor,
    row_scale: torch.Tensor | None = None, dest: torch.Tensor | None = None, num_dest_rows: int | None = None,
) -> torch.Tensor:
    """fp8 w2 GEMM + routing scale + scatter: out[dest[j]] = row_scale[j] * y[j]."""
    dev = _gpu("aq", aq)
    aq, sa_t, w2q, s2, M, H, E, D = _fp8_operands(aq, sa_t, w2q, s2, dev)
    offs = _offs(offs, dev)
    if row_scale is not None:
        row_scale = _want("row_scale", row_scale, torch.float32)
    if dest is not None:
        dest = _want("dest", dest, torch.int32)
    nd = M if num_dest_rows is None else int(num_dest_rows)
    out = torch.empty(nd, D, dtype=_BF16, device=dev)
    ws = _gemm_ws(M, E, dev)
    _lib.call(
        "ttamd_grouped_mm_fp8_unpermute", _p(aq), _p(sa_t), _p(w2q), _p(s2), _p(offs), M, E, D, H, _p(row_scale),
        _p(dest), nd, _p(out), _p(ws), ws.numel(), _stream(dev),
    )
    return out
