"""Checkpoint-format adapters of the fused expert weights (CPU only).

Layouts: reference / HipGroupedExperts w13 [E, 2H, D] gate-then-up and
w2 [E, D, H] (torchtitanturbo/models/common/npu_gmm.py:63-64); upstream
TorchTitan w1 / w3 [E, H, D]; Hugging Face per-expert gate/up/down_proj and
Llama4's input-major gate_up_proj / down_proj.
"""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

SD = importlib.import_module("torchtitan-ascend_amd.state_dict")
pkg = importlib.import_module("torchtitan-ascend_amd")
P = importlib.import_module("torchtitan-ascend_amd.protocol")


def _weights(E=3, D=16, H=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(E, H, D, generator=g), torch.randn(E, H, D, generator=g),
            torch.randn(E, D, H, generator=g))


def test_upstream_round_trip_and_values():
    w1, w3, w2 = _weights()
    sd = SD.upstream_to_fused({"moe.experts.w1": w1, "moe.experts.w3": w3, "moe.experts.w2": w2, "other": w2},
                              "moe.experts.")
    assert set(sd) == {"moe.experts.w13", "moe.experts.w2", "other"}
    H = w1.shape[1]
    assert torch.equal(sd["moe.experts.w13"][:, :H], w1) and torch.equal(sd["moe.experts.w13"][:, H:], w3)
    back = SD.fused_to_upstream(sd, "moe.experts.")
    assert torch.equal(back["moe.experts.w1"], w1) and torch.equal(back["moe.experts.w3"], w3)
    assert torch.equal(back["moe.experts.w2"], w2)


def test_fused_layout_computes_the_upstream_ffn():
    """silu(x w1^T) * (x w3^T) w2^T per expert equals the oracle's experts
    forward on the fused w13 (gate rows first): a swapped fuse fails."""
    w1, w3, w2 = _weights()
    E, H, D = w1.shape
    rng = np.random.default_rng(1)
    counts = np.array([4, 0, 5])
    x = rng.standard_normal((counts.sum(), D)).astype(np.float32)
    w13 = SD.fuse_w1_w3(w1, w3).numpy()
    y, _, _ = O.experts_forward(x, w13, w2.numpy(), counts, round_intermediates=False)
    ref = np.zeros_like(y)
    start = 0
    for e, c in enumerate(counts):
        xe = x[start:start + c].astype(np.float64)
        g = xe @ w1[e].double().numpy().T
        u = xe @ w3[e].double().numpy().T
        ref[start:start + c] = ((g / (1 + np.exp(-g))) * u) @ w2[e].double().numpy().T
        start += c
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)
    swapped = SD.fuse_w1_w3(w3, w1).numpy()
    y2, _, _ = O.experts_forward(x, swapped, w2.numpy(), counts, round_intermediates=False)
    assert not np.allclose(y2, ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("names", [("gate_proj", "up_proj", "down_proj"), ("w1", "w3", "w2")])
def test_hf_per_expert_round_trip(names):
    w1, w3, w2 = _weights(E=4)
    pre = "model.layers.3.mlp.experts."
    sd = {"model.layers.3.mlp.gate.weight": torch.zeros(4, 16)}
    for e in range(4):
        sd[f"{pre}{e}.{names[0]}.weight"] = w1[e]
        sd[f"{pre}{e}.{names[1]}.weight"] = w3[e]
        sd[f"{pre}{e}.{names[2]}.weight"] = w2[e]
    w13, w2f = SD.hf_experts_to_fused(sd, pre)
    assert torch.equal(w13, SD.fuse_w1_w3(w1, w3)) and torch.equal(w2f, w2)
    out = SD.fused_to_hf_experts(w13, w2f, pre)
    for e in range(4):
        assert torch.equal(out[f"{pre}{e}.gate_proj.weight"], w1[e])
        assert torch.equal(out[f"{pre}{e}.up_proj.weight"], w3[e])
        assert torch.equal(out[f"{pre}{e}.down_proj.weight"], w2[e])
    del sd[f"{pre}2.up_proj.weight" if names[1] == "up_proj" else f"{pre}2.w3.weight"]
    with pytest.raises(KeyError):
        SD.hf_experts_to_fused(sd, pre)


def test_hf_llama4_round_trip():
    w1, w3, w2 = _weights(E=2)
    w13 = SD.fuse_w1_w3(w1, w3)
    gate_up, down = SD.fused_to_hf_llama4(w13, w2)
    assert gate_up.shape == (2, 16, 16) and down.shape == (2, 8, 16)
    # Llama4 computes x @ gate_up_proj[e] -> [.., 2H], gate first
    x = torch.randn(5, 16, dtype=torch.float64)
    assert torch.allclose((x @ gate_up[0].double())[:, :8], x @ w1[0].double().T)
    w13b, w2b = SD.hf_llama4_to_fused(gate_up, down)
    assert torch.equal(w13b, w13) and torch.equal(w2b, w2)


def test_module_loads_upstream_checkpoint():
    """HipGroupedExperts.load_state_dict accepts upstream w1 / w3 keys."""
    E, D, H = 3, 16, 8
    cfg = pkg.HipGroupedExperts.Config(dim=D, hidden_dim=H, num_experts=E,
                                       token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=1))
    m = cfg.build()
    w1, w3, w2 = _weights(E, D, H)
    m.load_state_dict({"w1": w1, "w3": w3, "w2": w2})
    assert torch.equal(m.w13.data, SD.fuse_w1_w3(w1, w3)) and torch.equal(m.w2.data, w2)
    m.load_state_dict(m.state_dict())  # own format still loads
