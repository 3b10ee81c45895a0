"""The inference layer captured as one HIP graph (graph.MoELayerGraph):
every replay equals the eager two-call step on the same input, bit for bit,
with eager work and synchronisations between the replays (replays after the
first are where wrong graph nodes would show).  Shapes
(Llama4-debugmodel: T=2048, D=256, H=512, E=8, top-1 sigmoid, score before
the experts), a reduced Qwen3-30B-A3B layer (top-8 softmax + renorm) and a
layer whose w13 leftover tiles are split along k.
Reference: NpuGroupedExperts.forward with its router (npu_gmm.py:100-110)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, bf16_dev, rand_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,D,H,E,K,func,norm,before", [
    (2048, 256, 512, 8, 1, "sigmoid", False, True),
    (1024, 512, 256, 32, 8, "softmax", True, False),
    # w13: 64 tiles of 32 k stages on 256 CUs, each split into 4 pieces, so
    # the replays reuse the plan's arrival counters
    (1024, 2048, 1024, 8, 2, "softmax", True, False),
])
def test_graph_replays_equal_eager(ops, T, D, H, E, K, func, norm, before):
    G = importlib.import_module("torchtitan-ascend_amd.graph")
    rng = np.random.default_rng(T + K)
    wr = bf16_dev(rand_bf16(rng, (E, D), 0.02))
    w13 = bf16_dev(rand_bf16(rng, (E, 2 * H, D), 0.02))
    w2 = bf16_dev(rand_bf16(rng, (E, D, H), 0.02))

    def eager(x):
        _, _, r = ops.router_route(x, wr, K, func, norm, with_inverse=False)
        return ops.experts_forward(x, r, w13, w2, K, before)

    announce(f"graph capture T={T} D={D} H={H} E={E} K={K}")
    with torch.no_grad():
        layer = G.MoELayerGraph(bf16_dev(rand_bf16(rng, (T, D))), wr, w13, w2, K, func, norm, before)
        for i in range(4):
            x = bf16_dev(rand_bf16(rng, (T, D)))
            got = layer(x).clone()
            other = eager(bf16_dev(rand_bf16(rng, (T, D))))  # eager work between replays
            torch.cuda.synchronize()
            want = eager(x)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"replay {i} differs from the eager step"
            assert not torch.equal(other, want)
