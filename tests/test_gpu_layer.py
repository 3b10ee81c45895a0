"""GPU parity of the whole converted MoE expert layer (dispatch -> experts ->
combine) against the CPU oracle, forward and backward, including the
BASELINE configs at full size (checked on sampled tokens)."""
from __future__ import annotations

import importlib
import zlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, assert_dot_close, bf16_dev, edge_rows, f32_dev, rand_bf16, to_np, topk_labels
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _build(pkg, E, D, H, K, score_before, limit=None):
    P = __import__("importlib").import_module("torchtitan-ascend_amd.protocol")
    mc = P.ModelConfig()
    mc.layers = [P.GroupedExperts.Config(
        dim=D, hidden_dim=H, num_experts=E,
        token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K, score_before_experts=score_before),
    )]
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config(swiglu_limit=limit)).convert(mc)
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config()).convert(mc)
    return mc.layers[0].build()


def _inputs(rng, T, D, H, E, K, router="softmax", norm=True):
    x = rand_bf16(rng, (T, D))
    w13 = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2 = rand_bf16(rng, (E, D, H), 0.02)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    return x, w13, w2, logits


@pytest.mark.parametrize(
    "name,T,D,H,E,K,router,norm,score_before,limit",
    [
        ("c1_llama4_debug", 2048, 256, 512, 8, 1, "sigmoid", False, True, None),
        ("c2_qwen3_reduced", 512, 2048, 768, 128, 8, "softmax", True, False, None),
        ("limit_k2", 256, 256, 128, 8, 2, "softmax", True, False, 0.05),
    ],
)
def test_module_forward_vs_oracle(pkg, ops, name, T, D, H, E, K, router, norm, score_before, limit):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x, w13, w2, logits = _inputs(rng, T, D, H, E, K)
    announce(f"layer forward {name}")
    # the oracle routes with the GPU's choice (router parity is tested on its own)
    scores, idx = ops.router_topk(f32_dev(logits), K, router, norm)
    rs, ri = scores.cpu().numpy(), idx.cpu().numpy()
    m = _build(pkg, E, D, H, K, score_before, limit).to(DEV)
    with torch.no_grad():
        m.w13.copy_(bf16_dev(w13).float())
        m.w2.copy_(bf16_dev(w2).float())
    m = m.to(torch.bfloat16)
    with torch.no_grad():
        out = m(bf16_dev(x).view(1, T, D), scores, idx)
    ref = O.moe_forward(x, rs, ri, w13, w2, E, score_before, limit)
    assert out.shape == (T, D)
    assert_close(to_np(out), ref, TOL, f"layer output {name}")


@pytest.mark.parametrize("score_before,K,limit", [(False, 2, None), (True, 1, None), (False, 4, 0.05)])
def test_training_path_grads_vs_oracle(pkg, score_before, K, limit):
    rng = np.random.default_rng(100 + K)
    T, D, H, E = 256, 256, 128, 8
    x, w13, w2, _ = _inputs(rng, T, D, H, E, K)
    idx = topk_labels(T, K, E, rng)
    sc = (rng.random((T, K)) * 0.8 + 0.2).astype(np.float32)
    dout = rand_bf16(rng, (T, D))
    announce(f"training grads score_before={score_before} K={K} limit={limit}")
    m = _build(pkg, E, D, H, K, score_before, limit).to(DEV)
    with torch.no_grad():
        m.w13.copy_(f32_dev(w13))
        m.w2.copy_(f32_dev(w2))
    xd = bf16_dev(x).view(1, T, D).requires_grad_(True)
    sd = f32_dev(sc).requires_grad_(True)
    out = m(xd, sd, torch.from_numpy(idx).to(DEV))
    out.backward(bf16_dev(dout))
    ref_out = O.moe_forward(x, sc, idx, w13, w2, E, score_before, limit)
    # the kernels clamp the bf16 pre-activation, as the reference does
    ref = O.moe_backward(x, sc, idx, w13, w2, E, score_before, dout, limit, round_intermediates=True)
    assert_close(to_np(out), ref_out, TOL, "layer output")
    assert m.w13.grad.dtype == torch.float32
    assert_close(to_np(xd.grad).reshape(T, D), ref["dx"], TOL, "dX")
    assert O.max_rel_err(to_np(sd.grad), ref["dscores"]) < TOL
    assert_dot_close(to_np(sd.grad), ref["dscores"], ref["dscores_abs"], TOL, "d(top_scores)")
    assert_close(to_np(m.w13.grad), ref["dw13"], TOL, "dW13 (per expert)")
    assert_close(to_np(m.w2.grad), ref["dw2"], TOL, "dW2 (per expert)")


@pytest.mark.parametrize("limit", [None, 0.5])
def test_run_experts_grouped_mm_vs_oracle(limit):
    """The reference-signature entry (run_experts_grouped_mm, mirroring
    _run_experts_grouped_mm, npu_gmm.py:21-40) on its own, against the
    oracle: fp32 x (not bf16-representable, so the .bfloat16() cast at :31
    matters), fp32 weight Parameters (:63-64), the clamp (:32-36), empty
    experts, the output in x's dtype (:38 type_as), and its gradients
    (dx, dW13, dW2 in fp32; exact zeros for the experts without rows)."""
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(61)
    E, D, H = 8, 256, 128
    counts = np.array([37, 0, 250, 1, 0, 128, 300, 0])
    M = int(counts.sum())
    x = rng.standard_normal((M, D)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * H, D)) * 0.05).astype(np.float32)
    w2 = (rng.standard_normal((E, D, H)) * 0.05).astype(np.float32)
    dout = rand_bf16(rng, (M, D))
    xd = f32_dev(x).requires_grad_(True)
    w13d = f32_dev(w13).requires_grad_(True)
    w2d = f32_dev(w2).requires_grad_(True)
    announce(f"run_experts_grouped_mm fp32 x / weights, limit={limit}")
    y = F.run_experts_grouped_mm(w13d, w2d, xd, torch.from_numpy(counts).to(DEV), limit)
    assert y.dtype == torch.float32 and y.shape == (M, D)
    y.backward(f32_dev(dout))
    xb, w13b, w2b = O.bf16_round(x), O.bf16_round(w13), O.bf16_round(w2)
    ref_y, _, _ = O.experts_forward(xb, w13b, w2b, counts, limit)
    assert_close(to_np(y), ref_y, TOL, "y")
    # the same rows as a top-1 layer with unit scores applied before the
    # experts: routed rows already in expert order, so dispatch is the identity
    idx = np.repeat(np.arange(E), counts)[:, None].astype(np.int64)
    ref = O.moe_backward(xb, np.ones((M, 1), np.float32), idx, w13b, w2b, E, True, dout, limit,
                         round_intermediates=True)
    assert xd.grad.dtype == torch.float32 and w13d.grad.dtype == torch.float32 and w2d.grad.dtype == torch.float32
    assert_close(to_np(xd.grad), ref["dx"], TOL, "dx")
    assert_close(to_np(w13d.grad), ref["dw13"], TOL, "dW13 (per expert)")
    assert_close(to_np(w2d.grad), ref["dw2"], TOL, "dW2 (per expert)")
    for e in np.nonzero(counts == 0)[0]:
        assert not to_np(w13d.grad[e]).any() and not to_np(w2d.grad[e]).any(), f"empty expert {e}"


def test_dispatcher_api_matches_fused_forward(pkg):
    """dispatch -> _experts_forward -> combine (the reference's call chain,
    npu_gmm.py:100-110) gives the fused path's result."""
    rng = np.random.default_rng(7)
    T, D, H, E, K = 512, 512, 256, 16, 4
    x, w13, w2, _ = _inputs(rng, T, D, H, E, K)
    idx = torch.from_numpy(topk_labels(T, K, E, rng)).to(DEV)
    sc = f32_dev(rng.random((T, K)).astype(np.float32))
    m = _build(pkg, E, D, H, K, False).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        m.w13.copy_(bf16_dev(w13))
        m.w2.copy_(bf16_dev(w2))
        announce("dispatcher api vs fused")
        xb = bf16_dev(x)
        fused = m(xb.view(1, T, D), sc, idx)
        routed, counts, meta = m.token_dispatcher.dispatch(xb, sc, idx)
        y = m._experts_forward(routed, counts)
        composed = m.token_dispatcher.combine(y, meta, xb)
    assert O.max_rel_err(to_np(fused), to_np(composed)) < 1e-2


def _full_size_sampled(pkg, ops, T, D, H, E, K, router, norm, score_before, n_sample=48, labels=None):
    rng = np.random.default_rng(T + E)
    x = torch.randn(T, D, device=DEV).to(torch.bfloat16)
    m = _build(pkg, E, D, H, K, score_before).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        m.w13.normal_(0, 0.02)
        m.w2.normal_(0, 0.02)
    if labels is None:
        logits = torch.randn(T, E, device=DEV)
        scores, idx = ops.router_topk(logits, K, router, norm)
    else:
        idx = torch.from_numpy(labels.reshape(T, K)).to(DEV)
        scores = f32_dev(rng.random((T, K)).astype(np.float32))
    with torch.no_grad():
        out = m(x.view(1, T, D), scores, idx)
    # random tokens plus the tokens at the first / last row of every expert
    # segment and of every 32 / 256 / 320-row tile of the routed order
    idx_np = idx.cpu().numpy()
    sidx = O.stable_order(idx_np, E)
    edge_tok = sidx[edge_rows(np.cumsum(O.histogram(idx_np, E)))] // K
    rows = np.unique(np.concatenate([rng.choice(T, n_sample, replace=False), edge_tok]))
    rt = torch.from_numpy(rows).to(DEV)
    ix = idx_np[rows]
    ref = O.moe_forward(to_np(x[rt]), scores[rt].cpu().numpy(), ix, to_np(m.w13), to_np(m.w2), E, score_before)
    assert_close(to_np(out[rt]), ref, TOL, f"full-size layer output ({rows.size} sampled tokens)")
    return O.max_rel_err(to_np(out[rt]), ref)


def test_c2_qwen3_full_size_sampled(pkg, ops):
    announce("C2 full size")
    assert _full_size_sampled(pkg, ops, 8192, 2048, 768, 128, 8, "softmax", True, False) < TOL


def test_c4_deepseek_shard_full_size_sampled(pkg, ops):
    """32 local experts, D=7168, H=2048; 32768 routed rows (T=32768, K=1) with
    Zipf(1.2) expert load (largest ~10x mean, 4 experts empty)."""
    from gpu_util import labels_from_counts, zipf_counts

    rng = np.random.default_rng(44)
    labels = labels_from_counts(zipf_counts(32768, 32, 1.2, 28, rng), rng)
    announce("C4 full size")
    err = _full_size_sampled(pkg, ops, 32768, 7168, 2048, 32, 1, "sigmoid", False, False, n_sample=24, labels=labels)
    assert err < TOL


@pytest.mark.parametrize("T,D,H,gated,limit", [(300, 256, 128, True, None), (1000, 512, 192, False, None),
                                              (77, 128, 64, True, 0.4), (64, 128, 64, False, 0.0),
                                              # w2: 7 x 8 tiles of 64 k stages, split into 4 pieces
                                              # (the accumulating, gated epilogue runs once per tile)
                                              (2048, 2048, 4096, True, None)])
def test_shared_expert_add_vs_oracle(pkg, ops, T, D, H, gated, limit):
    """Shared expert fused into the combine (the shared w2 GEMM adds into the
    routed output in its epilogue) against the oracle's block tail."""
    rng = np.random.default_rng(T + D)
    x = rand_bf16(rng, (T, D))
    w13 = rand_bf16(rng, (2 * H, D), 0.08)
    w2 = rand_bf16(rng, (D, H), 0.08)
    routed = rand_bf16(rng, (T, D))
    gl = (rng.standard_normal(T) * 2).astype(np.float32) if gated else None
    announce(f"shared_expert_add T={T} D={D} H={H} gated={gated} limit={limit}")
    out = bf16_dev(routed)
    ops.shared_expert_add(out, bf16_dev(x), bf16_dev(w13), bf16_dev(w2),
                          None if gl is None else torch.from_numpy(gl).to(DEV), limit)
    ref = O.shared_expert_add(routed, x, w13, w2, gl, limit)
    assert_close(to_np(out), ref, 2e-2, "to_np(out)")
    # the functional form (no autograd: the fused pass) gives the same bits
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    with torch.no_grad():
        out2 = F.shared_expert_combine(bf16_dev(routed), bf16_dev(x), bf16_dev(w13), bf16_dev(w2),
                                       None if gl is None else torch.from_numpy(gl).to(DEV), limit)
    assert torch.equal(out2, out)
    # the autograd form clamps the same way (swiglu_limit=0.0 clamps to zero, None does not clamp)
    xr = bf16_dev(x).requires_grad_(True)
    out3 = F.shared_expert_combine(bf16_dev(routed), xr, bf16_dev(w13), bf16_dev(w2),
                                   None if gl is None else torch.from_numpy(gl).to(DEV), limit)
    assert O.max_rel_err(to_np(out3.detach()), to_np(out)) < 1e-2


def test_shared_expert_combine_autograd(pkg, ops):
    """With autograd the shared expert runs as a one-expert ttamd::experts and the
    gate in torch; forward matches the fused pass and gradients reach x,
    both shared weights, the gate logits and the routed output."""
    rng = np.random.default_rng(3)
    T, D, H = 200, 256, 128
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    x = bf16_dev(rand_bf16(rng, (T, D))).requires_grad_(True)
    w13 = bf16_dev(rand_bf16(rng, (2 * H, D), 0.08)).requires_grad_(True)
    w2 = bf16_dev(rand_bf16(rng, (D, H), 0.08)).requires_grad_(True)
    routed = bf16_dev(rand_bf16(rng, (T, D))).requires_grad_(True)
    gl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).to(DEV).requires_grad_(True)
    announce("shared_expert_combine autograd")
    out = F.shared_expert_combine(routed, x, w13, w2, gl)
    with torch.no_grad():
        fused = F.shared_expert_combine(routed, x, w13, w2, gl)
    assert O.max_rel_err(to_np(out.detach()), to_np(fused)) < 2e-2
    out.float().square().sum().backward()
    for name, t in (("x", x), ("w13", w13), ("w2", w2), ("gate_logits", gl), ("routed", routed)):
        assert t.grad is not None and torch.isfinite(t.grad.float()).all(), name
        assert t.grad.float().abs().sum() > 0, name
