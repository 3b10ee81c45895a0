"""The path's torch.library registration (torchtitan-ascend_amd/library.py):
torch.library.opcheck on every ttamd::* op (schema, fake tensor, autograd
registration, AOT dispatch with dynamic shapes), and the converted MoE layer
with its router under torch.compile(backend="aot_eager", fullgraph=True):
no graph break, and the compiled forward and backward give what eager gives,
bit for bit (the same HIP kernels run).  Reference: the traceable
torch._grouped_mm the reference calls (npu_gmm.py:17-18)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, bf16_dev, rand_bf16

pytestmark = pytest.mark.gpu

T, D, H, E, K = 40, 128, 128, 8, 2


def _routing():
    rng = np.random.default_rng(4)
    idx = torch.from_numpy(np.argsort(rng.random((T, E)), axis=1)[:, :K].astype(np.int64)).to(DEV)
    scores = torch.rand(T, K, device=DEV)
    counts, offsets, sidx, inv, ss = torch.ops.ttamd.route(idx.reshape(-1), E, scores.reshape(-1))
    return idx, scores, counts, offsets, sidx, inv, ss


def _cases():
    importlib.import_module("torchtitan-ascend_amd.library")
    rng = np.random.default_rng(5)
    x = bf16_dev(rand_bf16(rng, (T, D)))
    wr = bf16_dev(rand_bf16(rng, (E, D), 0.05))
    w13 = bf16_dev(rand_bf16(rng, (E, 2 * H, D), 0.05))
    w2 = bf16_dev(rand_bf16(rng, (E, D, H), 0.05))
    idx, scores, counts, offsets, sidx, inv, ss = _routing()
    sflat = scores.reshape(-1).contiguous()
    offs = offsets[1:].contiguous()
    M = T * K
    routed = bf16_dev(rand_bf16(rng, (M, D)))
    g = lambda *s: bf16_dev(rand_bf16(rng, s))  # noqa: E731
    _, _, logits = torch.ops.ttamd.router(x, wr, K, "softmax", True, 1.0, None, 1e-20)
    h = g(M, 2 * H)
    a = g(M, H)
    y = g(M, D)
    rq = lambda t: t.detach().clone().requires_grad_(True)  # noqa: E731
    return {
        "router": (torch.ops.ttamd.router, (rq(x), rq(wr), K, "softmax", True, 1.0, None, 1e-20)),
        "router_backward": (torch.ops.ttamd.router_backward,
                            (torch.randn(T, K, device=DEV), idx, logits, x, wr, "softmax", True, 1.0, 1e-20)),
        "route": (torch.ops.ttamd.route, (idx.reshape(-1), E, sflat)),
        "dispatch": (torch.ops.ttamd.dispatch, (rq(x), rq(sflat), sidx, inv, ss, K, True)),
        "dispatch_backward": (torch.ops.ttamd.dispatch_backward, (routed, x, sflat, sidx, inv, K, True)),
        "experts": (torch.ops.ttamd.experts, (rq(routed), rq(w13), rq(w2), offs, None, True)),
        # fp32 master weights: the op returns its bf16 copies for the backward
        "experts_fp32_weights": (torch.ops.ttamd.experts,
                                 (rq(routed), rq(w13.float()), rq(w2.float()), offs, 0.75, True)),
        "experts_backward": (torch.ops.ttamd.experts_backward,
                             (y, routed, h, a, w13, w2, offs, 0.75, True, True, True, torch.bfloat16,
                              torch.bfloat16)),
        "experts_backward_fp32_grads": (torch.ops.ttamd.experts_backward,
                                        (y, routed, h, a, w13, w2, offs, None, True, True, True, torch.float32,
                                         torch.float32)),
        "combine": (torch.ops.ttamd.combine, (rq(y), rq(sflat), sidx, inv, K, True)),
        "combine_backward": (torch.ops.ttamd.combine_backward, (x, y, sflat, sidx, K, True, True)),
        "moe_experts_forward": (torch.ops.ttamd.moe_experts_forward, (x, sidx, offsets, ss, w13, w2, K, False, None)),
        "shared_expert_add": (torch.ops.ttamd.shared_expert_add, (x, x, w13[0], w2[0], None, None)),
        "token_permute": (torch.ops.ttamd.token_permute, (rq(y), sidx.to(torch.int64) % E, E)),
        "token_unpermute": (torch.ops.ttamd.token_unpermute, (rq(y), sidx)),
        "token_gather": (torch.ops.ttamd.token_gather, (rq(y), sidx)),
    }


OP_NAMES = ["router", "router_backward", "route", "dispatch", "dispatch_backward", "experts", "experts_fp32_weights",
            "experts_backward", "experts_backward_fp32_grads", "combine", "combine_backward", "moe_experts_forward", "shared_expert_add", "token_permute",
            "token_unpermute", "token_gather"]


@pytest.mark.parametrize("name", OP_NAMES)
def test_opcheck(name):
    op, args = _cases()[name]
    announce(f"opcheck ttamd::{name}")
    torch.library.opcheck(op, args)


def _layer(pkg, score_before):
    P = importlib.import_module("torchtitan-ascend_amd.protocol")
    mc = P.ModelConfig()
    mc.layers = [P.GroupedExperts.Config(
        dim=D, hidden_dim=H, num_experts=E,
        token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K, score_before_experts=score_before),
    )]
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config()).convert(mc)
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config()).convert(mc)
    return mc.layers[0].build().to(DEV)


@pytest.mark.parametrize("score_before", [False, True])
def test_converted_layer_under_torch_compile(pkg, score_before):
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    torch.manual_seed(1)
    m = _layer(pkg, score_before)
    with torch.no_grad():
        m.w13.normal_(0, 0.05)
        m.w2.normal_(0, 0.05)
    m = m.to(torch.bfloat16)
    wr = (torch.randn(E, D, device=DEV) * 0.05).to(torch.bfloat16)
    x = torch.randn(1, T, D, device=DEV).to(torch.bfloat16)
    dout = torch.randn(T, D, device=DEV).to(torch.bfloat16)

    def layer(xx, w_router):
        scores, idx = F.router(xx, w_router, K, "softmax", True)
        return m(xx, scores, idx)

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    announce(f"torch.compile aot_eager converted layer, score_before={score_before}")
    grads = []
    outs = []
    for fn in (layer, compiled):
        m.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        wg = wr.clone().requires_grad_(True)
        out = fn(xg, wg)
        out.backward(dout)
        outs.append(out.detach())
        grads.append((xg.grad, wg.grad, m.w13.grad, m.w2.grad))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(*grads):
        assert a is not None and torch.equal(a, b)
    # inference (no autograd): the fused expert-stage op inside the graph
    with torch.no_grad():
        assert torch.equal(layer(x, wr), compiled(x, wr))
