"""CPU oracle of the MoE expert path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference path's algorithm, used as the checker
by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg.
Nothing in the product (torchtitan-ascend_amd/) imports it; the product
fails loudly without its HIP library instead of falling back to this code.

Each function cites the reference (file:line under torchtitanturbo/) or the
upstream TorchTitan behaviour it restates.  UPSTREAM marks TorchTitan code
that the reference calls but does not vendor; it is restated from its
public design.  How each function is pinned (the checks that do not merely
retype it) is listed in PINNED below and exercised by tests/test_oracle_*.py.

Numerics: inputs that are bf16 in the reference are converted exactly to
fp32 (bf16 -> fp32 is exact); products are accumulated in fp32 (float64 for
the reductions noted); values the reference materialises in bf16 (grouped
GEMM outputs, SwiGLU output, dispatch rows with the score multiply) are
rounded to bf16 at the same points, with round-to-nearest-even.
"""
from __future__ import annotations

import numpy as np

# Function -> how it is pinned (see tests/test_oracle_*.py).
PINNED = {
    "stable_order": "brute-force Python loop; torch.argsort(stable=True) golden vectors; hypothesis invariants",
    "histogram": "brute-force count; torch.bincount golden; sum == M",
    "permute / unpermute": "round trip unpermute(permute(x)) == x; torch index_select/index_add golden",
    "group_labels": "torch arange.repeat.repeat_interleave golden (npu_permute.py:68-72)",
    "router_topk": "torch softmax/sigmoid + topk golden on tie-free inputs; explicit tie cases; NaN golden "
                   "(torch.sort stable descending, same picks as torch.topk)",
    "router_logits": "torch F.linear (fp32) rounded to bf16 golden; exact bf16 values (a missing rounding or a "
                     "transposed weight fails it)",
    "experts_forward": "torch._grouped_mm golden; per-expert index_add loop and dense einsum forms",
    "moe_forward": "per-token brute loop of model.py:703-735 form",
    "shared_expert_add": "torch bf16 golden of the reference block's op sequence (FeedForward w1/w3/w2 Linear, "
                         "sigmoid(shared_expert_gate), expert_output + shared, model.py:794-809); a dropped gate "
                         "fails it",
    "moe_backward": "torch autograd of a torch fp32 restatement (golden); central finite differences",
    "router_backward": "torch CPU autograd of the upstream router op sequence (bf16 F.linear, fp32 softmax / "
                       "sigmoid, topk, renorm, route_scale) golden: dlogits, dx, dw; central finite differences "
                       "of router_forward_f64 (a dropped renorm term or a wrong softmax Jacobian fails them)",
    "grouped_dgrad / grouped_wgrad": "through moe_backward's autograd golden (they are its dx / dW steps); "
                                     "brute-force triple loop on tiny shapes",
    "swiglu_backward": "through moe_backward (above); finite differences of swiglu on clamped and unclamped "
                       "values; torch CPU autograd of torch.clamp + silu * up on NaN, +-inf, the limit and "
                       "signed zeros",
    "expert_weight_grad_slices": "equal to the matching slices of moe_backward's full dw13 / dw2 on small shapes "
                                 "(a swapped gate/up half or a transposed slice fails it)",
    "bf16_round": "torch .to(bfloat16) on random and special values",
    "f32_to_e4m3_bits / e4m3_bits_to_f32": "torch .to(float8_e4m3fn) on every bf16 bit pattern, ties and edge "
                                          "values; the 256-entry decode table vs torch float8 -> float",
    "quantize_fp8_rows / quantize_fp8_blocks": "torch float8 golden of the absmax/448 recipe; invariants: "
                                               "|q*s - v| <= half an e4m3 step of v, max |q| == 448 per block",
    "grouped_mm_fp8 / moe_forward_fp8": "grouped_mm (pinned above) on the dequantised operands; "
                                        "bf16 forward within fp8 error",
}


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even); NaN stays NaN."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------------------
# Routing (integer, bit-exact)
# ---------------------------------------------------------------------------
def histogram(labels: np.ndarray, num_experts: int) -> np.ndarray:
    """counts[e] = #{s : labels[s] == e}.  UPSTREAM dispatch:
    torch.histc(selected_experts_indices.view(-1), bins=E, min=0, max=E),
    consumed at npu_gmm.py:29; labels outside [0, E) are not counted."""
    lab = np.asarray(labels).reshape(-1).astype(np.int64)
    valid = (lab >= 0) & (lab < num_experts)
    return np.bincount(lab[valid], minlength=num_experts).astype(np.int32)


def stable_order(labels: np.ndarray, num_experts: int) -> np.ndarray:
    """Stable sort of the flat labels.  UPSTREAM dispatch:
    torch.argsort(selected_experts_indices.view(-1), stable=True); also the
    order torch_npu.npu_moe_token_permute produces (npu_permute.py:74-76).
    Labels outside [0, E) are placed after every valid label, in input order."""
    lab = np.asarray(labels).reshape(-1).astype(np.int64)
    bucket = np.where((lab >= 0) & (lab < num_experts), lab, num_experts)
    return np.argsort(bucket, kind="stable").astype(np.int32)


def inverse_order(sorted_indices: np.ndarray) -> np.ndarray:
    inv = np.empty_like(sorted_indices)
    inv[sorted_indices] = np.arange(sorted_indices.size, dtype=sorted_indices.dtype)
    return inv


def offsets_from_counts(counts: np.ndarray) -> np.ndarray:
    """Exclusive offsets [E+1]; offsets[1:] is the inclusive cumsum the
    reference passes to grouped_mm (npu_gmm.py:29)."""
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def permute(tokens: np.ndarray, labels: np.ndarray, top_k: int, num_experts: int):
    """npu_moe_token_permute(tokens, indices) (npu_permute.py:74-76):
    returns (permuted rows, sorted_indices) with permuted[j] = tokens[sorted[j] // K]."""
    sidx = stable_order(labels, num_experts)
    return np.asarray(tokens)[sidx // top_k], sidx


def unpermute(permuted: np.ndarray, sorted_indices: np.ndarray, probs: np.ndarray | None, top_k: int):
    """_npu_moe_token_unpermute_with_routing_map (npu_permute.py:23-30) and
    UPSTREAM combine: out[t] = sum_k w(t,k) * permuted[pos(t,k)], fp32
    accumulation in k order, bf16 result."""
    p = np.asarray(permuted, dtype=np.float32)
    M, D = p.shape
    T = M // top_k
    unsorted = np.empty_like(p)
    unsorted[sorted_indices] = p
    unsorted = unsorted.reshape(T, top_k, D)
    w = np.ones((T, top_k), np.float32) if probs is None else np.asarray(probs, np.float32).reshape(T, top_k)
    acc = np.zeros((T, D), np.float32)
    for k in range(top_k):
        acc += w[:, k, None] * unsorted[:, k]
    return bf16_round(acc)


def unpermute_grad(grad_out: np.ndarray, sorted_indices: np.ndarray, probs: np.ndarray | None, top_k: int,
                   permuted: np.ndarray | None = None):
    """npu_moe_token_unpermute_with_routing_map_grad (npu_permute.py:41-50):
    grad_permuted[j] = w(s) * grad_out[s // K], s = sorted[j]; optional
    grad_probs[s] = <grad_out[s // K], permuted[j]>."""
    g = np.asarray(grad_out, np.float32)
    s = np.asarray(sorted_indices)
    w = np.ones(s.size, np.float32) if probs is None else np.asarray(probs, np.float32).reshape(-1)[s]
    gp = bf16_round(g[s // top_k] * w[:, None])
    gprobs = None
    if permuted is not None:
        gprobs = np.zeros(s.size, np.float32)
        gprobs[s] = np.einsum("jd,jd->j", g[s // top_k].astype(np.float64),
                              np.asarray(permuted, np.float64)).astype(np.float32)
    return gp, gprobs


def group_labels(counts_group: np.ndarray, num_local_experts: int, num_rows: int) -> np.ndarray:
    """Labels of NpuTokenDispatcher._permute (npu_permute.py:68-72):
    arange(E_loc).repeat(ep).repeat_interleave(counts_group); rows past the
    total get label E_loc."""
    cg = np.asarray(counts_group).reshape(-1)
    ep = cg.size // num_local_experts
    lab = np.repeat(np.tile(np.arange(num_local_experts), ep), cg)
    out = np.full(num_rows, num_local_experts, dtype=np.int32)
    n = min(num_rows, lab.size)
    out[:n] = lab[:n]
    return out


def regroup_permute(routed_input: np.ndarray, counts_group: np.ndarray, ep_size: int, num_local_experts: int):
    """NpuTokenDispatcher._permute (npu_permute.py:63-85): stable regroup of
    rank-major rows into expert-major order.  Returns
    (permuted, permuted_indices, num_tokens_per_expert)."""
    labels = group_labels(counts_group, num_local_experts, routed_input.shape[0])
    permuted, sidx = permute(routed_input, labels, 1, num_local_experts)
    ntpe = np.asarray(counts_group).reshape(ep_size, -1).sum(0)
    return permuted, sidx, ntpe


# ---------------------------------------------------------------------------
# Router top-k (UPSTREAM TokenChoiceTopKRouter; closed form in the reference
# at models/qwen3_5/model.py:757-765)
# ---------------------------------------------------------------------------
def router_logits(x: np.ndarray, w_router: np.ndarray) -> np.ndarray:
    """Router gate logits F.linear(x, weight) in bf16 (models/qwen3_5/model.py:757;
    UPSTREAM TokenChoiceTopKRouter.gate is a bias-free nn.Linear): the bf16
    inputs accumulated in float64, rounded once to bf16 (via fp32)."""
    z = np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T
    return bf16_round(z.astype(np.float32))


def router_topk(logits: np.ndarray, top_k: int, score_func: str = "softmax", route_norm: bool = False,
                route_scale: float = 1.0, expert_bias: np.ndarray | None = None, norm_eps: float = 1e-20):
    """Scores in fp32 (softmax over experts or sigmoid); pick the top_k by
    score (+ expert_bias for selection only), descending with NaN first (as
    torch.topk ranks it), ties to the lower expert id; optional renormalisation by the sum of the picked scores
    (model.py:762-764, UPSTREAM adds norm_eps); multiply by route_scale."""
    z = np.asarray(logits, np.float32)
    if score_func == "softmax":
        m = z.max(axis=-1, keepdims=True)
        e = np.exp((z - m).astype(np.float64))
        s = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    elif score_func == "sigmoid":
        s = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    else:
        raise ValueError(score_func)
    sel = s if expert_bias is None else s + np.asarray(expert_bias, np.float32)
    T, E = s.shape
    # lexsort (last key primary): NaN before every number (torch.topk ranks
    # NaN as the largest value), then -sel (descending), then the expert id
    # (ascending): the order of torch.sort(sel, descending=True, stable=True)
    isnan = np.isnan(sel)
    neg = np.where(isnan, 0.0, -sel)
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), neg, ~isnan), axis=-1)[:, :top_k]
    top = np.take_along_axis(s, order, axis=-1).astype(np.float64)
    if route_norm:
        top = top / (top.sum(axis=-1, keepdims=True) + norm_eps)
    top = top * route_scale
    return top.astype(np.float32), order.astype(np.int64)


def router_scores(logits: np.ndarray, score_func: str) -> np.ndarray:
    """fp32 expert scores of the router: softmax over experts or sigmoid
    (models/qwen3_5/model.py:758; UPSTREAM sigmoid)."""
    z = np.asarray(logits, np.float32)
    if score_func == "softmax":
        m = z.max(axis=-1, keepdims=True)
        e = np.exp((z - m).astype(np.float64))
        return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    if score_func == "sigmoid":
        return (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    raise ValueError(score_func)


def router_backward(x: np.ndarray, w_router: np.ndarray, logits: np.ndarray, idx: np.ndarray,
                    grad_top: np.ndarray, score_func: str = "softmax", route_norm: bool = False,
                    route_scale: float = 1.0, norm_eps: float = 1e-20, round_bf16: bool = True):
    """Autograd of the router forward (UPSTREAM TokenChoiceTopKRouter; closed
    form models/qwen3_5/model.py:757-765): logits = x w^T (bf16 Linear),
    s = softmax / sigmoid(logits) in fp32, top = s[idx] (renormalised by
    sum + eps when route_norm) * route_scale.  Given d(top) [T, K] and the
    picks idx (selection has no gradient; expert_bias only steers it):
        ds[idx_k] = g_k / S - sum_j g_j s_j / S^2  (renorm),  g_k otherwise
        dz = (ds - <ds, s>) s  (softmax)  or  ds (1 - s) s  (sigmoid)
        dlogits = bf16(dz)   (the gradient of the bf16 logits)
        dx = dlogits w,  dw = dlogits^T x   (float64 accumulation)
    Returns (dx, dw, dlogits) in fp32; with round_bf16=False nothing is
    rounded (the smooth function finite differences see)."""
    s = router_scores(logits, score_func).astype(np.float64)
    T, E = s.shape
    idx = np.asarray(idx, np.int64).reshape(T, -1)
    g = np.asarray(grad_top, np.float64).reshape(T, -1) * route_scale
    picked = np.take_along_axis(s, idx, axis=-1)
    if route_norm:
        S = picked.sum(-1, keepdims=True) + norm_eps
        ds_k = g / S - (g * picked).sum(-1, keepdims=True) / (S * S)
    else:
        ds_k = g
    ds = np.zeros((T, E))
    np.add.at(ds, (np.arange(T)[:, None], idx), ds_k)
    if score_func == "softmax":
        dz = (ds - (ds * s).sum(-1, keepdims=True)) * s
    else:
        dz = ds * (1.0 - s) * s
    dlog = bf16_round(dz.astype(np.float32)) if round_bf16 else dz
    dx = np.asarray(dlog, np.float64) @ np.asarray(w_router, np.float64)
    dw = np.asarray(dlog, np.float64).T @ np.asarray(x, np.float64)
    return dx.astype(np.float32), dw.astype(np.float32), np.asarray(dlog, np.float32)


def router_forward_f64(x: np.ndarray, w_router: np.ndarray, idx: np.ndarray, score_func: str,
                       route_norm: bool, route_scale: float, norm_eps: float = 1e-20) -> np.ndarray:
    """The router forward in float64 with fixed picks and no bf16 rounding:
    the smooth function router_backward(round_bf16=False) differentiates
    (for finite-difference checks)."""
    z = np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T
    if score_func == "softmax":
        e = np.exp(z - z.max(-1, keepdims=True))
        s = e / e.sum(-1, keepdims=True)
    else:
        s = 1.0 / (1.0 + np.exp(-z))
    top = np.take_along_axis(s, np.asarray(idx, np.int64), axis=-1)
    if route_norm:
        top = top / (top.sum(-1, keepdims=True) + norm_eps)
    return top * route_scale


# ---------------------------------------------------------------------------
# Expert FFN (npu_gmm.py:21-40)
# ---------------------------------------------------------------------------
def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    with np.errstate(invalid="ignore", over="ignore"):  # silu(-inf) is NaN, as in torch
        return (x / (1.0 + np.exp(-x))).astype(np.float32)


def grouped_mm(x: np.ndarray, w: np.ndarray, offs: np.ndarray) -> np.ndarray:
    """torch._grouped_mm(x, w.transpose(-2, -1), offs) (npu_gmm.py:17-18):
    out[m] = x[m] @ w[e(m)]^T for m in [offs[e-1], offs[e]), fp32 accumulate.
    Rows past offs[-1] are left at zero."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    out = np.zeros((x.shape[0], w.shape[1]), np.float32)
    start = 0
    for e, end in enumerate(np.asarray(offs).tolist()):
        if end > start:
            out[start:end] = x[start:end] @ w[e].T
        start = end
    return out


def grouped_dgrad(dy: np.ndarray, w: np.ndarray, offs: np.ndarray) -> np.ndarray:
    """Backward of grouped_mm w.r.t. x (autograd of torch._grouped_mm,
    npu_gmm.py:31, :38): dx[m] = dy[m] @ w[e(m)], w [E, N, K]; fp32
    accumulate; rows past offs[-1] are zero."""
    dy = np.asarray(dy, np.float32)
    w = np.asarray(w, np.float32)
    dx = np.zeros((dy.shape[0], w.shape[2]), np.float32)
    start = 0
    for e, end in enumerate(np.asarray(offs).tolist()):
        if end > start:
            dx[start:end] = dy[start:end] @ w[e]
        start = end
    return dx


def grouped_wgrad(dy: np.ndarray, x: np.ndarray, offs: np.ndarray, num_experts: int) -> np.ndarray:
    """Backward of grouped_mm w.r.t. the weight: dw[e] = dy_e^T @ x_e over
    expert e's rows [offs[e-1], offs[e]); an expert without rows gets exact
    zeros.  dy [M, N], x [M, K] -> dw [E, N, K], fp32 accumulate."""
    dy = np.asarray(dy, np.float32)
    x = np.asarray(x, np.float32)
    dw = np.zeros((num_experts, dy.shape[1], x.shape[1]), np.float32)
    start = 0
    for e, end in enumerate(np.asarray(offs).tolist()):
        if end > start:
            dw[e] = dy[start:end].T @ x[start:end]
        start = end
    return dw


def swiglu(h: np.ndarray, swiglu_limit: float | None = None) -> np.ndarray:
    """Clamp (npu_gmm.py:32-36) then npu_swiglu (npu_gmm.py:37):
    gate = first half, up = second half; silu(gate) * up."""
    H = h.shape[-1] // 2
    gate, up = h[..., :H], h[..., H:]
    if swiglu_limit is not None:
        up = np.clip(up, -swiglu_limit, swiglu_limit)
        gate = np.minimum(gate, swiglu_limit)
    return (silu(gate) * up).astype(np.float32)


def experts_forward(x: np.ndarray, w13: np.ndarray, w2: np.ndarray, counts: np.ndarray,
                    swiglu_limit: float | None = None, round_intermediates: bool = True):
    """_run_experts_grouped_mm (npu_gmm.py:21-40) on routed rows x [M, D].
    Returns (y [M, D], h [M, 2H], a [M, H]); with round_intermediates the
    grouped GEMM outputs and the SwiGLU output are rounded to bf16 where the
    reference materialises them in bf16."""
    offs = np.cumsum(counts).astype(np.int64)
    h = grouped_mm(x, w13, offs)
    if round_intermediates:
        h = bf16_round(h)
    a = swiglu(h, swiglu_limit)
    if round_intermediates:
        a = bf16_round(a)
    y = grouped_mm(a, w2, offs)
    if round_intermediates:
        y = bf16_round(y)
    return y, h, a


def shared_expert_add(routed_out: np.ndarray, x: np.ndarray, w13s: np.ndarray, w2s: np.ndarray,
                      gate_logits: np.ndarray | None = None, swiglu_limit: float | None = None) -> np.ndarray:
    """Shared expert added to the combined routed output
    (models/qwen3_5/model.py:794-809; UPSTREAM Llama4 MoE: out + shared_experts(x)):
      y     = FeedForward(x): silu(x w1^T) * (x w3^T), then w2, each Linear
              output in bf16 (w1 / w3 are the gate / up halves of w13s [2H, D]);
      g     = sigmoid(gate_logits) in bf16 (Linear(D, 1) output, :804-807), or 1;
      out   = bf16(routed_out + bf16(g * y))                         (:808)."""
    T = x.shape[0]
    y, _, _ = experts_forward(x, w13s[None], w2s[None], np.array([T]), swiglu_limit)
    if gate_logits is not None:
        g = bf16_round((1.0 / (1.0 + np.exp(-np.asarray(gate_logits, np.float64)))).astype(np.float32))
        y = bf16_round(g.reshape(T, 1) * y)
    return bf16_round(np.asarray(routed_out, np.float32) + y)


def moe_forward(x: np.ndarray, top_scores: np.ndarray, idx: np.ndarray, w13: np.ndarray, w2: np.ndarray,
                num_experts: int, score_before_experts: bool, swiglu_limit: float | None = None,
                round_intermediates: bool = True) -> np.ndarray:
    """NpuGroupedExperts.forward (npu_gmm.py:100-110): UPSTREAM dispatch
    (gather in stable expert order, fp32 score multiply before the experts
    if score_before_experts), experts, UPSTREAM combine (score multiply after
    the experts otherwise, K-way sum).  x [T, D] -> [T, D]."""
    T, D = x.shape
    K = top_scores.shape[-1]
    flat_scores = np.asarray(top_scores, np.float32).reshape(-1)
    sidx = stable_order(idx, num_experts)
    counts = histogram(idx, num_experts)
    routed = np.asarray(x, np.float32)[sidx // K]
    if score_before_experts:
        routed = routed * flat_scores[sidx][:, None]
        if round_intermediates:
            routed = bf16_round(routed)
    y, _, _ = experts_forward(routed, w13, w2, counts, swiglu_limit, round_intermediates)
    probs = None if score_before_experts else flat_scores
    return unpermute(y, sidx, probs, K) if round_intermediates else _unpermute_f32(y, sidx, probs, K)


def _unpermute_f32(y, sidx, probs, K):
    M, D = y.shape
    un = np.empty_like(y)
    un[sidx] = y
    un = un.reshape(M // K, K, D)
    w = np.ones((M // K, K), np.float32) if probs is None else probs.reshape(M // K, K)
    return (un * w[..., None]).sum(1).astype(np.float32)


def moe_backward(x, top_scores, idx, w13, w2, num_experts, score_before_experts, dout,
                 swiglu_limit: float | None = None, round_intermediates: bool = False):
    """Gradients of moe_forward: returns dict(dx [T,D], dscores [T,K],
    dw13 [E,2H,D], dw2 [E,D,H]).  The chain is the autograd of
    npu_gmm.py:21-40 plus the UPSTREAM dispatch/combine score multiplies.

    Gradients are accumulated in fp32.  With round_intermediates the forward
    values the reference materialises in bf16 are rounded where it rounds
    them: the dispatched rows (score before experts), the grouped_mm output
    h (npu_gmm.py:31; the clamp masks of :32-36 are taken from this bf16 h),
    the SwiGLU output a (:37) and the w2 output y (:38)."""
    rnd = bf16_round if round_intermediates else (lambda v: v)
    x = np.asarray(x, np.float32)
    T, D = x.shape
    K = top_scores.shape[-1]
    E = num_experts
    H = w2.shape[-1]
    s_flat = np.asarray(top_scores, np.float32).reshape(-1)
    sidx = stable_order(idx, E)
    counts = histogram(idx, E)
    offs = np.cumsum(counts)
    tok = sidx // K
    xr = x[tok]
    routed = rnd(xr * s_flat[sidx][:, None]) if score_before_experts else xr
    h = rnd(grouped_mm(routed, w13, offs))
    a = rnd(swiglu(h, swiglu_limit))
    y = rnd(grouped_mm(a, w2, offs))
    dout = np.asarray(dout, np.float32)
    g_tok = dout[tok]  # dOut gathered per routed row
    dscores = np.zeros(T * K, np.float32)
    if score_before_experts:
        dy = g_tok
    else:
        dy = g_tok * s_flat[sidx][:, None]
        dscores[sidx] = np.einsum("jd,jd->j", g_tok.astype(np.float64), y.astype(np.float64))
    dw2 = grouped_wgrad(dy, a, offs, E)
    da = grouped_dgrad(dy, w2, offs)
    dh = swiglu_backward(da, h, swiglu_limit)
    dw13 = grouped_wgrad(dh, routed, offs, E)
    d_routed = grouped_dgrad(dh, w13, offs)
    dx = np.zeros_like(x)
    # sum_d |a_d b_d| of each score gradient's dot product <a, b>: the scale
    # its rounding error is bounded by (tests compare per element against it)
    dscores_abs = np.zeros(T * K, np.float32)
    if score_before_experts:
        dscores[sidx] = np.einsum("jd,jd->j", d_routed.astype(np.float64), xr.astype(np.float64))
        dscores_abs[sidx] = np.einsum("jd,jd->j", np.abs(d_routed).astype(np.float64), np.abs(xr).astype(np.float64))
        np.add.at(dx, tok, d_routed * s_flat[sidx][:, None])
    else:
        dscores_abs[sidx] = np.einsum("jd,jd->j", np.abs(g_tok).astype(np.float64), np.abs(y).astype(np.float64))
        np.add.at(dx, tok, d_routed)
    return {"dx": dx, "dscores": dscores.reshape(T, K), "dscores_abs": dscores_abs.reshape(T, K),
            "dw13": dw13, "dw2": dw2}


def swiglu_backward(da: np.ndarray, h: np.ndarray, swiglu_limit: float | None = None) -> np.ndarray:
    """Gradient of swiglu(clamp(h)) (npu_gmm.py:32-37) w.r.t. the
    pre-activation h = [gate | up], given da = d(activation).  torch.clamp's
    backward is where(min <= h <= max, grad, 0): exactly zero where it
    clamped and where h is NaN, whatever the incoming gradient holds.
    Returns dh [.., 2H] = [[gate <= L] ? da * up_c * silu'(gate_c) : 0,
    [-L <= up <= L] ? da * silu(gate_c) : 0]."""
    H = h.shape[-1] // 2
    gate, up = h[..., :H], h[..., H:]
    gc, uc = gate, up
    if swiglu_limit is not None:
        gc = np.minimum(gate, swiglu_limit)
        uc = np.clip(up, -swiglu_limit, swiglu_limit)
    with np.errstate(invalid="ignore", over="ignore"):
        sig = (1.0 / (1.0 + np.exp(-gc.astype(np.float64)))).astype(np.float32)
        dsilu = sig * (1.0 + gc * (1.0 - sig))
        dgate = da * uc * dsilu
        dup = da * gc * sig
        if swiglu_limit is not None:
            dgate = np.where(gate <= swiglu_limit, dgate, np.float32(0))
            dup = np.where((up >= -swiglu_limit) & (up <= swiglu_limit), dup, np.float32(0))
    return np.concatenate([dgate, dup], axis=-1).astype(np.float32)


def expert_weight_grad_slices(routed: np.ndarray, dy: np.ndarray, w13_e: np.ndarray, w2_e: np.ndarray,
                              gate_rows: np.ndarray, down_cols: np.ndarray, swiglu_limit: float | None = None,
                              round_intermediates: bool = True):
    """Selected slices of ONE expert's weight gradients under
    _run_experts_grouped_mm's autograd (npu_gmm.py:31-38), without forming
    the whole [2H, D] / [D, H] gradients: the gradient of gate row n needs
    only columns n and H + n of the pre-activation, and column p of dW2 only
    column p of the activation.
      routed [n, D]: the expert's dispatched rows; dy [n, D]: gradient of
      its output rows; w13_e [2H, D]; w2_e [D, H].
    Returns (dw13_gate [len(gate_rows), D] = dW13[gate_rows],
             dw13_up [len(gate_rows), D] = dW13[H + gate_rows],
             dw2_cols [D, len(down_cols)] = dW2[:, down_cols]),
    with the bf16 roundings of moe_backward(round_intermediates=...)."""
    rnd = bf16_round if round_intermediates else (lambda v: v)
    r = np.asarray(routed, np.float32)
    g = np.asarray(dy, np.float32)
    w13_e = np.asarray(w13_e, np.float32)
    w2_e = np.asarray(w2_e, np.float32)
    H = w2_e.shape[1]
    gate_rows = np.asarray(gate_rows, np.int64)
    down_cols = np.asarray(down_cols, np.int64)
    h_sel = rnd(np.concatenate([r @ w13_e[gate_rows].T, r @ w13_e[H + gate_rows].T], axis=1))
    da_sel = g @ w2_e[:, gate_rows]
    dh_sel = swiglu_backward(da_sel, h_sel, swiglu_limit)
    ng = gate_rows.size
    dw13_gate = dh_sel[:, :ng].T @ r
    dw13_up = dh_sel[:, ng:].T @ r
    h_p = rnd(np.concatenate([r @ w13_e[down_cols].T, r @ w13_e[H + down_cols].T], axis=1))
    a_p = rnd(swiglu(h_p, swiglu_limit))
    dw2_cols = g.T @ a_p
    return dw13_gate.astype(np.float32), dw13_up.astype(np.float32), dw2_cols.astype(np.float32)


# ---------------------------------------------------------------------------
# fp8 e4m3 with block scales (not in the reference, which
# has no fp8 path: the published recipe is restated -- s = absmax / 448 per
# block, q = e4m3fn(v / s), dequantised value q * s, GEMM in fp32).
# ---------------------------------------------------------------------------
FP8_MAX = 448.0
FP8_BLOCK = 128


def f32_to_e4m3_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> OCP float8 e4m3fn bits (bias 7, no infinities), round to
    nearest even.  Magnitudes above 464 (half-way to the non-existent 480),
    infinities and NaN give NaN (0x7f | sign), as torch.float8_e4m3fn does.
    Computed in float64 from the decomposed value (exact), not by bit tricks."""
    a = np.asarray(a, np.float32)
    sign = ((a.view(np.uint32) >> 31).astype(np.uint8) << 7)
    with np.errstate(invalid="ignore"):
        v = np.abs(a.astype(np.float64))
    nan = ~(v <= 464.0)  # NaN, inf and > 464
    v = np.where(nan, 0.0, v)
    # exponent of the result's quantum: normals 2^(e-3), subnormals 2^-9
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(v > 0, v, 1.0)))
    e = np.clip(e, -6, 8)
    quantum = np.exp2(e - 3)
    r = np.rint(v / quantum) * quantum  # exact: v / quantum has <= 24 significant bits
    # encode r (0 <= r <= 448)
    with np.errstate(divide="ignore"):
        er = np.floor(np.log2(np.where(r > 0, r, 1.0)))
    normal = r >= 2.0 ** -6
    exp_field = np.where(normal, er + 7, 0)
    mant = np.where(normal, r / np.exp2(er) - 1.0, r / 2.0 ** -9) * np.where(normal, 8.0, 1.0)
    bits = (exp_field.astype(np.int64) << 3) | np.rint(mant).astype(np.int64)
    bits = np.where(nan, 0x7F, bits).astype(np.uint8)
    return bits | sign


def _e4m3_table() -> np.ndarray:
    t = np.zeros(256, np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 0xF and m == 7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * m * 2.0 ** -9
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_VALUES = _e4m3_table()


def e4m3_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return E4M3_VALUES[np.asarray(bits, np.uint8)]


def _block_quant(v: np.ndarray, axis_block_shape) -> tuple[np.ndarray, np.ndarray]:
    """Quantise v (float32, already reshaped so that the block elements span
    the axes in axis_block_shape) -> (bits, scale).  scale = absmax / 448 in
    fp32; q = e4m3(v / scale) with the fp32 quotient; an all-zero block has
    scale 0 and codes 0."""
    amax = np.max(np.abs(v), axis=axis_block_shape, keepdims=True).astype(np.float32)
    scale = (amax / np.float32(FP8_MAX)).astype(np.float32)
    safe = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    q = (v / safe).astype(np.float32)
    bits = np.where(scale > 0, f32_to_e4m3_bits(q), np.uint8(0)).astype(np.uint8)
    return bits, scale


def quantize_fp8_rows(x: np.ndarray, block: int = FP8_BLOCK) -> tuple[np.ndarray, np.ndarray]:
    """Activations: per row, per `block` consecutive channels.
    x [R, K] -> (bits uint8 [R, K], scale fp32 [R, K / block])."""
    x = np.asarray(x, np.float32)
    R, K = x.shape
    v = x.reshape(R, K // block, block)
    bits, scale = _block_quant(v, (2,))
    return bits.reshape(R, K), scale.reshape(R, K // block)


def quantize_fp8_blocks(w: np.ndarray, block: int = FP8_BLOCK) -> tuple[np.ndarray, np.ndarray]:
    """Weights: per block x block tile of each expert matrix.
    w [E, N, K] -> (bits uint8 [E, N, K], scale fp32 [E, N / block, K / block])."""
    w = np.asarray(w, np.float32)
    E, N, K = w.shape
    v = w.reshape(E, N // block, block, K // block, block)
    bits, scale = _block_quant(v, (2, 4))
    return (bits.reshape(E, N, K), scale.reshape(E, N // block, K // block))


def dequant_rows(bits: np.ndarray, scale: np.ndarray, block: int = FP8_BLOCK) -> np.ndarray:
    R, K = bits.shape
    return (e4m3_bits_to_f32(bits).reshape(R, K // block, block) * scale[:, :, None]).reshape(R, K)


def dequant_blocks(bits: np.ndarray, scale: np.ndarray, block: int = FP8_BLOCK) -> np.ndarray:
    E, N, K = bits.shape
    v = e4m3_bits_to_f32(bits).reshape(E, N // block, block, K // block, block)
    return (v * scale[:, :, None, :, None]).reshape(E, N, K)


def grouped_mm_fp8(xq, sx, wq, sw, offs) -> np.ndarray:
    """fp8 grouped GEMM: dequantise both operands (q * s) and run the fp32
    grouped GEMM.  xq [M, K], sx [M, K/128], wq [E, N, K], sw [E, N/128, K/128]."""
    return grouped_mm(dequant_rows(xq, sx), dequant_blocks(wq, sw), offs)


def moe_forward_fp8(x, top_scores, idx, w13q, s13, w2q, s2, num_experts, score_before_experts,
                    swiglu_limit=None):
    """moe_forward with fp8 experts: the dispatched rows
    are quantised per token and 128 channels, w13/w2 are pre-quantised with
    128 x 128 block scales, h and a are materialised in bf16 as in the bf16
    path, and the SwiGLU output is re-quantised per row for the w2 GEMM."""
    T, D = x.shape
    K = top_scores.shape[-1]
    flat_scores = np.asarray(top_scores, np.float32).reshape(-1)
    sidx = stable_order(idx, num_experts)
    counts = histogram(idx, num_experts)
    offs = np.cumsum(counts).astype(np.int64)
    routed = np.asarray(x, np.float32)[sidx // K]
    if score_before_experts:
        routed = bf16_round(routed * flat_scores[sidx][:, None])
    xq, sx = quantize_fp8_rows(routed)
    h = bf16_round(grouped_mm_fp8(xq, sx, w13q, s13, offs))
    a = bf16_round(swiglu(h, swiglu_limit))
    aq, sa = quantize_fp8_rows(a)
    y = bf16_round(grouped_mm_fp8(aq, sa, w2q, s2, offs))
    probs = None if score_before_experts else flat_scores
    return unpermute(y, sidx, probs, K)


def max_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the norm-wise relative error the
    tolerances 2e-2 / 5e-2 are stated in)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.abs(ref).max()
    if denom == 0:
        return float(np.abs(got).max())
    return float(np.abs(got - ref).max() / denom)
