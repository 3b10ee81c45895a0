"""Seeded random sweep of the path over the options the fixed cases pin one
at a time: ragged token counts, expert counts that are not powers of two,
top-k from 1 to 8, softmax or sigmoid with or without renormalisation and
expert bias, score before or after the experts, the SwiGLU clamp on or off,
experts without rows, and model / hidden sizes from the smallest the C ABI
takes upward.

* Inference (ttamd_router_route + ttamd_moe_experts_forward): the dispatch
  order and histogram bit-exact against the oracle (stable_order,
  histogram) on the router's own picks, the layer output within the path's
  2e-2 per token row (models/qwen3_5/model.py:752-766, npu_gmm.py:21-40 and
  :100-110, npu_permute.py:23-30).
* Training (the converted module under autograd): output, dX, d(top_scores)
  and per-expert dW13 / dW2 against the oracle's backward (npu_gmm.py:31,
  :38 under autograd, npu_permute.py:35-53).

Each case names its seed and shape before it runs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, assert_dot_close, bf16_dev, f32_dev, rand_bf16, to_np, topk_labels
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _fwd_case(seed: int) -> dict:
    rng = np.random.default_rng(7100 + seed)
    E = int(rng.integers(1, 41))
    return dict(
        T=int(rng.integers(1, 700)),
        D=int(rng.choice([128, 256, 384, 640, 1024])),
        H=int(rng.choice([64, 128, 192, 320, 512])),
        E=E,
        K=int(rng.integers(1, min(E, 8) + 1)),
        func=str(rng.choice(["softmax", "sigmoid"])),
        norm=bool(rng.integers(0, 2)),
        bias=bool(rng.integers(0, 2)),
        before=bool(rng.integers(0, 2)),
        limit=[None, 0.5, 2.0][int(rng.integers(0, 3))],
    )


EDGE_CASES = [
    # one token, one expert; the largest expert count with top-8 over few
    # tokens (most experts empty); two experts holding ~1000 rows each
    dict(T=1, D=128, H=64, E=1, K=1, func="sigmoid", norm=False, bias=False, before=False, limit=None),
    dict(T=3, D=128, H=64, E=256, K=8, func="softmax", norm=True, bias=True, before=False, limit=None),
    dict(T=1000, D=256, H=64, E=2, K=2, func="softmax", norm=True, bias=False, before=False, limit=0.5),
]


@pytest.mark.parametrize("seed", range(16 + len(EDGE_CASES)))
def test_sweep_inference_vs_oracle(ops, seed):
    c = _fwd_case(seed) if seed < 16 else EDGE_CASES[seed - 16]
    T, D, H, E, K = c["T"], c["D"], c["H"], c["E"], c["K"]
    rng = np.random.default_rng(seed)
    xh = rand_bf16(rng, (T, D))
    w13h = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2h = rand_bf16(rng, (E, D, H), 0.02)
    wr = bf16_dev(rand_bf16(rng, (E, D), 0.05))
    eb = f32_dev((rng.standard_normal(E) * 0.01).astype(np.float32)) if c["bias"] else None
    announce(f"sweep inference seed={seed} {c}")
    s, i, r = ops.router_route(bf16_dev(xh), wr, K, c["func"], c["norm"], 1.0, eb)
    out = ops.experts_forward(bf16_dev(xh), r, bf16_dev(w13h), bf16_dev(w2h), K, c["before"], c["limit"])
    torch.cuda.synchronize()
    idx = i.cpu().numpy()
    assert idx.shape == (T, K) and idx.min() >= 0 and idx.max() < E
    assert all(len(set(row)) == K for row in idx.tolist()), "a token picked one expert twice"
    np.testing.assert_array_equal(r.counts.cpu().numpy(), O.histogram(idx, E))
    np.testing.assert_array_equal(r.sorted_indices.cpu().numpy(), O.stable_order(idx, E))
    ref = O.moe_forward(xh, s.cpu().numpy(), idx, w13h, w2h, E, c["before"], swiglu_limit=c["limit"])
    assert out.shape == (T, D)
    assert_close(to_np(out), ref, TOL, f"sweep seed {seed} output")


def _build(pkg, E, D, H, K, score_before, limit):
    import importlib

    P = importlib.import_module("torchtitan-ascend_amd.protocol")
    mc = P.ModelConfig()
    mc.layers = [P.GroupedExperts.Config(
        dim=D, hidden_dim=H, num_experts=E,
        token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K, score_before_experts=score_before),
    )]
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config(swiglu_limit=limit)).convert(mc)
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config()).convert(mc)
    return mc.layers[0].build()


@pytest.mark.parametrize("seed", range(6))
def test_sweep_training_vs_oracle(pkg, seed):
    rng = np.random.default_rng(7300 + seed)
    E = int(rng.integers(2, 25))
    K = int(rng.integers(1, min(E, 4) + 1))
    T = int(rng.integers(8, 400))
    D = int(rng.choice([128, 256, 384, 512]))
    H = int(rng.choice([128, 256, 384]))  # training takes H % 128 == 0
    before = bool(rng.integers(0, 2))
    limit = [None, 0.5][int(rng.integers(0, 2))]
    x = rand_bf16(rng, (T, D))
    w13 = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2 = rand_bf16(rng, (E, D, H), 0.02)
    idx = topk_labels(T, K, E, rng)
    sc = (rng.random((T, K)) * 0.8 + 0.2).astype(np.float32)
    dout = rand_bf16(rng, (T, D))
    announce(f"sweep training seed={seed} T={T} D={D} H={H} E={E} K={K} before={before} limit={limit}")
    m = _build(pkg, E, D, H, K, before, limit).to(DEV)
    with torch.no_grad():
        m.w13.copy_(f32_dev(w13))
        m.w2.copy_(f32_dev(w2))
    xd = bf16_dev(x).view(1, T, D).requires_grad_(True)
    sd = f32_dev(sc).requires_grad_(True)
    out = m(xd, sd, torch.from_numpy(idx).to(DEV))
    out.backward(bf16_dev(dout))
    torch.cuda.synchronize()
    ref_out = O.moe_forward(x, sc, idx, w13, w2, E, before, limit)
    ref = O.moe_backward(x, sc, idx, w13, w2, E, before, dout, limit, round_intermediates=True)
    assert_close(to_np(out), ref_out, TOL, "output")
    assert_close(to_np(xd.grad).reshape(T, D), ref["dx"], TOL, "dX")
    assert_dot_close(to_np(sd.grad), ref["dscores"], ref["dscores_abs"], TOL, "d(top_scores)")
    assert_close(to_np(m.w13.grad), ref["dw13"], TOL, "dW13 (per expert)")
    assert_close(to_np(m.w2.grad), ref["dw2"], TOL, "dW2 (per expert)")
    empty = np.setdiff1d(np.arange(E), np.unique(idx))
    for e in empty:
        assert not to_np(m.w13.grad[e]).any() and not to_np(m.w2.grad[e]).any(), f"expert {e} without rows"
