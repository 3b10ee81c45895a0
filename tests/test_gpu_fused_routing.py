"""GPU parity of the fused router + dispatch order (ttamd_router_route) and
of the one-call expert stage (ttamd_moe_experts_forward).

ttamd_router_route must give exactly what ttamd_router_fused followed by
ttamd_moe_route gives on its picks (the same kernels, fused launches):
scores, expert ids, counts, offsets, stable order, inverse, sorted scores,
bit for bit; its tile plan must equal the table the host-side rule below
derives from the counts; tokens_per_expert must grow by the histogram of the
picks (oracle.histogram), call after call.  ttamd_moe_experts_forward must
match the stage-by-stage inference path bit for bit and the CPU oracle to
the path's 2e-2 (per row).  Reference: models/qwen3_5/model.py:752-766
(router), npu_gmm.py:100-110 with :21-40 (experts), npu_permute.py:23-30
(combine)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, rand_bf16, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2


def plan_table(counts: np.ndarray, M: int, max_rows: int = 320) -> tuple[int, np.ndarray]:
    """The token-tile table of the forward grouped GEMMs from per-expert row
    counts: an expert's c rows in n = ceil(c / max_rows) tiles of one height
    h = roundup32(ceil(c / n)), the last one shorter; tiles in expert order;
    M // 128 + E + 1 entries, those past the count {-1, 0, 0, 0}."""
    E = counts.size
    max_tiles = M // 128 + E + 1
    tab = np.tile(np.array([-1, 0, 0, 0], np.int32), (max_tiles, 1))
    i, r0 = 0, 0
    for e in range(E):
        c = int(counts[e])
        if c > 0:
            n0 = -(-c // max_rows)
            h = (-(-c // n0) + 31) // 32 * 32
            for t in range(-(-c // h)):
                tab[i] = (e, r0 + t * h, min(r0 + (t + 1) * h, r0 + c), 0)
                i += 1
        r0 += c
    return i, tab


# plan layout: int4 header {count, ...}, 512 split-tile counters, the table
SPLIT_TILES = 512
TABLE_OFF = 16 + 4 * SPLIT_TILES


def _plan_of(plan: torch.Tensor, M: int, E: int) -> tuple[int, np.ndarray]:
    raw = plan.cpu().numpy()
    max_tiles = M // 128 + E + 1
    assert not raw[16:TABLE_OFF].any(), "split-tile counters must be zero"
    return int(raw[:4].view(np.int32)[0]), raw[TABLE_OFF:TABLE_OFF + 16 * max_tiles].view(np.int32).reshape(max_tiles, 4)


ROUTER_CASES = [
    # T, D, E, K, score, renorm, bias
    (8192, 2048, 128, 8, "softmax", True, False),   # C2, Qwen3-30B-A3B (fused scan: 129 x 64 entries)
    (8192, 5120, 16, 1, "sigmoid", False, False),   # C3, Llama4-Scout router
    (4096, 1024, 256, 8, "sigmoid", True, True),    # DeepSeek-V3-like: 256 experts, load-balancing bias
    (37, 128, 6, 3, "softmax", False, True),        # ragged tiny case, 3 chunks of nothing
    (65536, 256, 256, 8, "softmax", True, False),   # 257 x 512 histogram: the separate-scan fallback
]


@pytest.mark.parametrize("T,D,E,K,func,norm,bias", ROUTER_CASES)
def test_router_route_matches_router_then_route(ops, T, D, E, K, func, norm, bias):
    rng = np.random.default_rng(T + E + K)
    x = bf16_dev(rand_bf16(rng, (T, D)))
    w = bf16_dev(rand_bf16(rng, (E, D), 0.02))
    eb = torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32)).to(DEV) if bias else None
    tpe0 = rng.random(E).astype(np.float32) * 100
    tpe = torch.from_numpy(tpe0.copy()).to(DEV)
    announce(f"router_route T={T} D={D} E={E} K={K} {func}")
    s, i, r = ops.router_route(x, w, K, func, norm, 1.0, eb, tokens_per_expert=tpe)
    s2, i2 = ops.router_fused(x, w, K, func, norm, 1.0, eb)
    r2 = ops.route(i2, E, s2)
    torch.cuda.synchronize()
    assert torch.equal(i, i2)
    assert torch.equal(s, s2)
    for name in ("counts", "offsets", "sorted_indices", "inverse", "sorted_scores"):
        np.testing.assert_array_equal(getattr(r, name).cpu().numpy(), getattr(r2, name).cpu().numpy(), err_msg=name)
    counts = O.histogram(i.cpu().numpy(), E)
    np.testing.assert_array_equal(r.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(r.sorted_indices.cpu().numpy(), O.stable_order(i.cpu().numpy(), E))
    # tile plan of the expert-sorted rows
    n, tab = _plan_of(r.plan, T * K, E)
    n_ref, tab_ref = plan_table(counts, T * K)
    assert n == n_ref
    np.testing.assert_array_equal(tab, tab_ref)
    # tokens_per_expert accumulates the histogram, call after call
    np.testing.assert_array_equal(tpe.cpu().numpy(), tpe0 + counts.astype(np.float32))
    ops.router_route(x, w, K, func, norm, 1.0, eb, tokens_per_expert=tpe)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(tpe.cpu().numpy(), (tpe0 + counts.astype(np.float32)) + counts.astype(np.float32))


def test_router_route_no_tokens(ops):
    E, D, K = 8, 128, 2
    x = torch.empty(0, D, dtype=torch.bfloat16, device=DEV)
    w = bf16_dev(rand_bf16(np.random.default_rng(0), (E, D), 0.02))
    tpe = torch.ones(E, device=DEV)
    announce("router_route T=0")
    s, i, r = ops.router_route(x, w, K, "softmax", True, tokens_per_expert=tpe)
    torch.cuda.synchronize()
    assert s.shape == (0, K) and i.shape == (0, K)
    assert not r.counts.cpu().numpy().any() and not r.offsets.cpu().numpy().any()
    assert _plan_of(r.plan, 0, E)[0] == 0
    assert torch.equal(tpe, torch.ones(E, device=DEV))


EXPERT_CASES = [
    # T, D, H, E, K, score_before, limit
    (512, 256, 128, 16, 8, False, None),   # C2-like: top-8, score after, gather fused into w13
    (300, 256, 192, 4, 1, True, None),     # C1/C3-like: top-1, score before (permute first)
    (257, 384, 128, 8, 2, False, 0.75),    # clamp, ragged T
    (200, 256, 64, 6, 3, True, None),      # score before with top-k > 1
]


@pytest.mark.parametrize("use_plan", [True, False])
@pytest.mark.parametrize("T,D,H,E,K,before,limit", EXPERT_CASES)
def test_experts_forward_matches_stages_and_oracle(ops, T, D, H, E, K, before, limit, use_plan):
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(T * 7 + K)
    xh = rand_bf16(rng, (T, D))
    w13h = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2h = rand_bf16(rng, (E, D, H), 0.02)
    wr = bf16_dev(rand_bf16(rng, (E, D), 0.02))
    x, w13, w2 = bf16_dev(xh), bf16_dev(w13h), bf16_dev(w2h)
    announce(f"experts_forward T={T} D={D} H={H} E={E} K={K} before={before} plan={use_plan}")
    s, i, r = ops.router_route(x, wr, K, "softmax", True)
    if not use_plan:
        r.plan = None
    out = ops.experts_forward(x, r, w13, w2, K, before, limit)
    with torch.no_grad():  # stage_events: the op-at-a-time path over the same kernels
        ref_stages = F.moe_experts_forward(x, s, i, w13, w2, E, before, limit, stage_events={})
    torch.cuda.synchronize()
    assert torch.equal(out, ref_stages), "one-call expert stage differs from the stage-by-stage path"
    ref = O.moe_forward(xh, s.cpu().numpy(), i.cpu().numpy(), w13h, w2h, E, before, swiglu_limit=limit)
    assert_close(to_np(out), ref, TOL, "experts_forward vs oracle")


def test_experts_forward_c2_full_size_matches_stages(ops):
    """Qwen3-30B-A3B at full size (T=8192, D=2048, H=768, E=128, top-8): the
    one-call stage with router_route's plan equals the stage-by-stage path."""
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    torch.manual_seed(0)
    T, D, H, E, K = 8192, 2048, 768, 128, 8
    x = torch.randn(T, D, device=DEV).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * H, D, device=DEV) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, D, H, device=DEV) * 0.02).to(torch.bfloat16)
    wr = (torch.randn(E, D, device=DEV) * 0.02).to(torch.bfloat16)
    announce("experts_forward C2 full size")
    s, i, r = ops.router_route(x, wr, K, "softmax", True)
    out = ops.experts_forward(x, r, w13, w2, K, False)
    with torch.no_grad():
        ref = F.moe_experts_forward(x, s, i, w13, w2, E, False, stage_events={})
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
