"""GPU parity of the router backward (ttamd_router_backward, ttamd::router's registered backward)
against the CPU oracle, itself pinned to torch autograd of the upstream
router op sequence (models/qwen3_5/model.py:757-765 closed form).

The oracle is fed the GPU forward's own picks and bf16 logits, so the check
is of the backward alone: dx [T, D] per token row and dW_r [E, D] per expert
row, each within the path's 2e-2 (norm-wise and per row)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, rand_bf16, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2

CASES = [
    # T, D, E, K, score, renorm, route_scale
    (8192, 2048, 128, 8, "softmax", True, 1.0),   # C2 router (Qwen3-30B-A3B)
    (8192, 5120, 16, 1, "sigmoid", False, 1.0),   # C3 router (Llama4-Scout)
    (2048, 1024, 256, 8, "sigmoid", True, 2.5),   # DeepSeek-V3-like: 256 experts, route_scale
    (333, 256, 40, 3, "softmax", False, 1.0),     # ragged: E not a multiple of 128, T not of 16
]


@pytest.mark.parametrize("T,D,E,K,func,norm,scale", CASES)
def test_router_backward_matches_oracle(ops, T, D, E, K, func, norm, scale):
    rng = np.random.default_rng(T + E)
    xh = rand_bf16(rng, (T, D))
    wh = rand_bf16(rng, (E, D), 0.02)
    g = rng.standard_normal((T, K)).astype(np.float32)
    x, w = bf16_dev(xh), bf16_dev(wh)
    announce(f"router backward T={T} D={D} E={E} K={K} {func} norm={norm}")
    s, idx, logits = ops.router_fused(x, w, K, func, norm, scale, return_logits=True)
    dx, dw = ops.router_backward(torch.from_numpy(g).to(DEV), idx, logits, x, w, func, norm, scale)
    torch.cuda.synchronize()
    rdx, rdw, _ = O.router_backward(xh, wh, to_np(logits), idx.cpu().numpy(), g, func, norm, scale)
    assert_close(to_np(dx), rdx, TOL, "router dx")
    assert_close(to_np(dw), rdw, TOL, "router dW")


def test_router_autograd(ops):
    """functional.router: the forward equals ttamd_router_fused bit for bit,
    and autograd delivers ttamd_router_backward's dx, dW (fp32 weight keeps
    an fp32 gradient, bf16 a bf16 one)."""
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(9)
    T, D, E, K = 1000, 512, 64, 4
    x = bf16_dev(rand_bf16(rng, (T, D)))
    w32 = torch.from_numpy(rand_bf16(rng, (E, D), 0.02)).to(DEV)
    g = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(DEV)
    announce("router autograd")
    for w_param in (w32.clone(), w32.to(torch.bfloat16)):
        xg = x.clone().requires_grad_(True)
        wg = w_param.clone().requires_grad_(True)
        s, i = F.router(xg, wg, K, "softmax", True)
        s2, i2, lg = ops.router_fused(x, w32.to(torch.bfloat16), K, "softmax", True, return_logits=True)
        assert torch.equal(s, s2) and torch.equal(i, i2)
        assert not i.requires_grad
        s.backward(g)
        dx, dw = ops.router_backward(g, i2, lg, x, w32.to(torch.bfloat16), "softmax", True, 1.0,
                                     dw_dtype=wg.dtype)
        torch.cuda.synchronize()
        assert wg.grad.dtype == wg.dtype
        assert torch.equal(xg.grad, dx)
        assert torch.equal(wg.grad, dw)
