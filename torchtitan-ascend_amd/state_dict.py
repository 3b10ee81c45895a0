"""Checkpoint-format adapters for the fused expert weights.

HipGroupedExperts keeps the reference's parameters (npu_gmm.py:63-64):
    w13 [E, 2H, D]   rows 0..H-1 = gate (w1), rows H..2H-1 = up (w3)
    w2  [E, D, H]
Checkpoints come in other layouts:
  * upstream TorchTitan GroupedExperts: w1 [E, H, D], w3 [E, H, D], w2 [E, D, H];
  * Hugging Face per-expert Linear weights (Qwen3-MoE, DeepSeek-V3, Mixtral
    naming): experts.{e}.gate_proj.weight [H, D], up_proj [H, D],
    down_proj [D, H];
  * Hugging Face Llama4 fused experts: gate_up_proj [E, D, 2H] (gate first),
    down_proj [E, H, D] (both stored input-major, i.e. transposed).

The functions here convert in both directions without changing values, so
a model converted with HipGroupedExpertsConverter loads and saves any of
them.  They run on whatever device the tensors are on (host code, not a
kernel: a checkpoint conversion is a one-off copy).
"""
from __future__ import annotations

import re

import torch

__all__ = [
    "fuse_w1_w3",
    "split_w13",
    "upstream_to_fused",
    "fused_to_upstream",
    "hf_experts_to_fused",
    "fused_to_hf_experts",
    "hf_llama4_to_fused",
    "fused_to_hf_llama4",
]


def fuse_w1_w3(w1: torch.Tensor, w3: torch.Tensor) -> torch.Tensor:
    """w1, w3 [E, H, D] -> w13 [E, 2H, D] (gate rows first)."""
    if w1.shape != w3.shape or w1.dim() != 3:
        raise ValueError(f"w1 and w3 must both be [E, H, D], got {tuple(w1.shape)} and {tuple(w3.shape)}")
    return torch.cat([w1, w3], dim=1)


def split_w13(w13: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w13 [E, 2H, D] -> (w1, w3) [E, H, D] (contiguous copies)."""
    if w13.dim() != 3 or w13.shape[1] % 2:
        raise ValueError(f"w13 must be [E, 2H, D], got {tuple(w13.shape)}")
    H = w13.shape[1] // 2
    return w13[:, :H].contiguous(), w13[:, H:].contiguous()


def upstream_to_fused(state_dict: dict, prefix: str = "") -> dict:
    """Replace {prefix}w1 / {prefix}w3 by {prefix}w13 in a state dict (other
    keys, w2 included, are kept).  A dict that already holds w13 is returned
    unchanged."""
    k1, k3, k13 = prefix + "w1", prefix + "w3", prefix + "w13"
    if k13 in state_dict or k1 not in state_dict:
        return dict(state_dict)
    if k3 not in state_dict:
        raise KeyError(f"{k1} present without {k3}")
    out = {k: v for k, v in state_dict.items() if k not in (k1, k3)}
    out[k13] = fuse_w1_w3(state_dict[k1], state_dict[k3])
    return out


def fused_to_upstream(state_dict: dict, prefix: str = "") -> dict:
    """Replace {prefix}w13 by {prefix}w1 / {prefix}w3."""
    k13 = prefix + "w13"
    if k13 not in state_dict:
        return dict(state_dict)
    out = {k: v for k, v in state_dict.items() if k != k13}
    out[prefix + "w1"], out[prefix + "w3"] = split_w13(state_dict[k13])
    return out


_HF_EXPERT = re.compile(r"^(?P<pre>.*experts\.)(?P<e>\d+)\.(?P<name>gate_proj|up_proj|down_proj|w1|w2|w3)\.weight$")
# Mixtral names its per-expert Linear layers w1 (gate), w3 (up), w2 (down).
_HF_ALIAS = {"w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}


def hf_experts_to_fused(state_dict: dict, experts_prefix: str) -> tuple[torch.Tensor, torch.Tensor]:
    """Collect experts_prefix + "{e}.gate_proj/up_proj/down_proj.weight" (or
    Mixtral's w1/w3/w2) into (w13 [E, 2H, D], w2 [E, D, H]).  Every expert
    0..E-1 must be present."""
    per: dict[int, dict[str, torch.Tensor]] = {}
    for key, val in state_dict.items():
        if not key.startswith(experts_prefix):
            continue
        m = _HF_EXPERT.match(key)
        if not m or m.group("pre") != experts_prefix:
            continue
        name = _HF_ALIAS.get(m.group("name"), m.group("name"))
        per.setdefault(int(m.group("e")), {})[name] = val
    if not per:
        raise KeyError(f"no expert weights under {experts_prefix!r}")
    E = max(per) + 1
    missing = [e for e in range(E) if set(per.get(e, {})) != {"gate_proj", "up_proj", "down_proj"}]
    if missing:
        raise KeyError(f"incomplete experts under {experts_prefix!r}: {missing[:8]}")
    w13 = torch.stack([torch.cat([per[e]["gate_proj"], per[e]["up_proj"]], dim=0) for e in range(E)])
    w2 = torch.stack([per[e]["down_proj"] for e in range(E)])
    return w13, w2


def fused_to_hf_experts(w13: torch.Tensor, w2: torch.Tensor, experts_prefix: str) -> dict:
    """(w13 [E, 2H, D], w2 [E, D, H]) -> experts_prefix + "{e}.{gate,up,down}_proj.weight"."""
    w1, w3 = split_w13(w13)
    out = {}
    for e in range(w13.shape[0]):
        out[f"{experts_prefix}{e}.gate_proj.weight"] = w1[e]
        out[f"{experts_prefix}{e}.up_proj.weight"] = w3[e]
        out[f"{experts_prefix}{e}.down_proj.weight"] = w2[e].contiguous()
    return out


def hf_llama4_to_fused(gate_up_proj: torch.Tensor, down_proj: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Llama4 fused experts, gate_up_proj [E, D, 2H] and down_proj [E, H, D]
    (input-major), -> (w13 [E, 2H, D], w2 [E, D, H])."""
    if gate_up_proj.dim() != 3 or down_proj.dim() != 3 or gate_up_proj.shape[2] % 2:
        raise ValueError("gate_up_proj must be [E, D, 2H] and down_proj [E, H, D]")
    return gate_up_proj.transpose(1, 2).contiguous(), down_proj.transpose(1, 2).contiguous()


def fused_to_hf_llama4(w13: torch.Tensor, w2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(w13 [E, 2H, D], w2 [E, D, H]) -> (gate_up_proj [E, D, 2H], down_proj [E, H, D])."""
    return w13.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
