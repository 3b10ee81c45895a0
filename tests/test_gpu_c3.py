"""BASELINE config 3 at full size: the Llama4-Scout-shaped MoE layer forward
+ backward (T=8192, D=5120, H=8192, E=16, top-1 sigmoid router, score before
the experts, plus one always-on shared expert of the same shape), through
the converted HipGroupedExperts layer and the shared-expert combine, with
autograd, against the CPU oracle.

Checked (tolerance: the path's 2e-2, norm-wise AND per row / per slice):
  * layer output and dX on >= 256 sampled tokens, including the first and
    last routed row of every expert segment and of every 32/256/320-row tile;
  * d(top_scores) of those tokens, per element against the dot-product
    error scale sum |a b|;
  * dW13 and dW2 in full for two experts (oracle on those experts' rows);
  * for every other expert, ~32 gate rows (+ their up rows) of dW13 and ~32
    columns of dW2, one or two in each of its 256-wide n / k tiles;
  * the shared expert's dW13 rows / dW2 columns likewise;
  * the router (differentiated with the layer): its share of dX on the
    sampled tokens and the router weight gradient dW_r [E, D].
Reference: autograd through torch._grouped_mm (npu_gmm.py:21-40) and the
unpermute (npu_permute.py:35-53); shared expert as models/qwen3_5/model.py
:794-809 without the gate (UPSTREAM Llama4)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, assert_dot_close, edge_rows, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2
T, D, H, E, K = 8192, 5120, 8192, 16, 1


def _build(pkg):
    P = importlib.import_module("torchtitan-ascend_amd.protocol")
    mc = P.ModelConfig()
    mc.layers = [P.GroupedExperts.Config(
        dim=D, hidden_dim=H, num_experts=E,
        token_dispatcher=P.AllToAllTokenDispatcher.Config(num_experts=E, top_k=K, score_before_experts=True),
    )]
    pkg.HipGroupedExpertsConverter(pkg.HipGroupedExpertsConverter.Config()).convert(mc)
    pkg.HipTokenDispatcherConverter(pkg.HipTokenDispatcherConverter.Config()).convert(mc)
    return mc.layers[0].build()


def _spread(n_total: int, count: int, rng, tile: int = 256) -> np.ndarray:
    """`count` indices of [0, n_total) covering every 256-wide tile."""
    n_tiles = -(-n_total // tile)
    per = -(-count // n_tiles)
    out = []
    for t in range(n_tiles):
        lo, hi = t * tile, min(n_total, (t + 1) * tile)
        out += [lo, hi - 1] + list(rng.integers(lo, hi, max(0, per - 2)))
    out = np.unique(np.asarray(out))
    return out if out.size <= count else np.unique(np.concatenate([out[:: max(1, out.size // count)], out[-1:]]))


@pytest.mark.timeout(900)
@pytest.mark.parametrize("param_dtype", ["bf16", "fp32"])
def test_c3_llama4_scout_fwd_bwd_full_size(pkg, ops, param_dtype):
    """param_dtype fp32: the expert weights (routed and shared) are fp32
    nn.Parameters as in the reference (npu_gmm.py:63-64), used in bf16 by the
    GEMMs (:31, :38: cast once per step, the forward's copy serving the
    backward) and given fp32 gradients; the oracle sees the bf16-rounded
    weights the reference's GEMMs see."""
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    torch.manual_seed(3)
    rng = np.random.default_rng(3)
    announce(f"C3 full size ({param_dtype} parameters): set-up")
    wdt = torch.float32 if param_dtype == "fp32" else torch.bfloat16
    x = torch.randn(T, D, device=DEV).to(torch.bfloat16)
    w_router = (torch.randn(E, D, device=DEV) * 0.02).to(torch.bfloat16)
    m = _build(pkg).to(DEV).to(wdt)
    with torch.no_grad():
        m.w13.normal_(0, 0.02)
        m.w2.normal_(0, 0.02)
    sw13 = (torch.randn(2 * H, D, device=DEV) * 0.02).to(wdt).requires_grad_(True)
    sw2 = (torch.randn(D, H, device=DEV) * 0.02).to(wdt).requires_grad_(True)
    dout = torch.randn(T, D, device=DEV).to(torch.bfloat16)
    assert m.w13.dtype == wdt and m.w2.dtype == wdt

    def wnp(t):  # the weights as the GEMMs see them (bf16)
        return O.bf16_round(to_np(t))

    announce(f"C3 full size ({param_dtype} parameters): router + layer forward + backward on the GPU")
    # the router is part of the differentiated graph: x and w_router get its
    # gradient too (scores.grad is kept to check d(top_scores))
    xg = x.clone().requires_grad_(True)
    wr = w_router.clone().requires_grad_(True)
    sc, idx = F.router(xg, wr, K, "sigmoid", False)
    sc.retain_grad()
    with torch.no_grad():
        _, _, logits = ops.router_fused(x, w_router, K, "sigmoid", False, return_logits=True)
    out = m(xg.view(1, T, D), sc, idx)
    out = F.shared_expert_combine(out, xg, sw13, sw2)
    out.backward(dout)
    torch.cuda.synchronize()
    for p_ in (m.w13, m.w2, sw13, sw2):
        assert p_.grad.dtype == wdt

    announce("C3 full size: oracle")
    idx_np = idx.cpu().numpy()
    sc_np = sc.detach().cpu().numpy()
    counts = O.histogram(idx_np, E)
    offs = np.cumsum(counts)
    assert counts.sum() == T and (counts > 0).all()
    sidx = O.stable_order(idx_np, E)
    # sampled tokens: every segment / tile edge of the routed order, plus random ones
    edge_tok = sidx[edge_rows(offs)] // K
    tok = np.unique(np.concatenate([edge_tok, rng.choice(T, 256, replace=False)]))
    assert tok.size >= 256
    tt = torch.from_numpy(tok).to(DEV)
    x_s = to_np(x[tt])
    dout_s = to_np(dout[tt])
    w13_all = m.w13.detach()
    w2_all = m.w2.detach()

    # shared expert (one expert with every token): its part of the sampled outputs and dX
    sw13_np, sw2_np = wnp(sw13), wnp(sw2)
    ones = np.ones((tok.size, 1), np.float32)
    zeros = np.zeros((tok.size, 1), np.int64)
    sh = O.moe_backward(x_s, ones, zeros, sw13_np[None], sw2_np[None], 1, True, dout_s, round_intermediates=True)
    sh_y = O.moe_forward(x_s, ones, zeros, sw13_np[None], sw2_np[None], 1, True)

    # routed experts: the oracle on the sampled tokens, one expert's weights at a time
    routed_y = np.zeros((tok.size, D), np.float32)
    dx_routed = np.zeros((tok.size, D), np.float32)
    ds = np.zeros((tok.size, K), np.float32)
    ds_abs = np.zeros((tok.size, K), np.float32)
    e_tok = idx_np[tok, 0]
    full_experts = [int(np.argmin(counts)), int(np.argmax(counts))]
    for e in range(E):
        announce(f"C3 full size: oracle, expert {e}")
        sel = np.nonzero(e_tok == e)[0]
        w13e, w2e = wnp(w13_all[e])[None], wnp(w2_all[e])[None]
        if sel.size:
            z = np.zeros((sel.size, 1), np.int64)
            routed_y[sel] = O.moe_forward(x_s[sel], sc_np[tok[sel]], z, w13e, w2e, 1, True)
            g = O.moe_backward(x_s[sel], sc_np[tok[sel]], z, w13e, w2e, 1, True, dout_s[sel], round_intermediates=True)
            dx_routed[sel], ds[sel], ds_abs[sel] = g["dx"], g["dscores"], g["dscores_abs"]
        # this expert's rows (in stable order) for its weight gradients
        rows = sidx[(offs[e] - counts[e]):offs[e]] // K
        rt = torch.from_numpy(rows).to(DEV)
        xe = to_np(x[rt])
        se = sc_np[rows]
        routed_e = O.bf16_round(xe * se)
        dy_e = to_np(dout[rt])
        got13, got2 = m.w13.grad[e], m.w2.grad[e]
        if e in full_experts:
            announce(f"C3 full size: full dW of expert {e} ({rows.size} rows)")
            g = O.moe_backward(xe, se, np.zeros((rows.size, 1), np.int64), w13e, w2e, 1, True, dy_e,
                               round_intermediates=True)
            assert_close(to_np(got13), g["dw13"][0], TOL, f"dW13 expert {e}")
            assert_close(to_np(got2), g["dw2"][0], TOL, f"dW2 expert {e}")
        else:
            gr = _spread(H, 32, rng)
            dc = _spread(H, 32, rng)
            g13, u13, c2 = O.expert_weight_grad_slices(routed_e, dy_e, w13e[0], w2e[0], gr, dc)
            assert_close(to_np(got13[torch.from_numpy(gr).to(DEV)]), g13, TOL, f"dW13 gate rows expert {e}")
            assert_close(to_np(got13[torch.from_numpy(H + gr).to(DEV)]), u13, TOL, f"dW13 up rows expert {e}")
            assert_close(to_np(got2[:, torch.from_numpy(dc).to(DEV)]).T, c2.T, TOL, f"dW2 columns expert {e}")

    ref_out = O.bf16_round(routed_y + sh_y)
    assert_close(to_np(out[tt]), ref_out, TOL, "layer output (sampled tokens)")
    assert_dot_close(to_np(sc.grad[tt]), ds, ds_abs, TOL, "d(top_scores) (sampled tokens)")
    # the router's share of dX on the sampled tokens, from the oracle's d(top_scores)
    lg = to_np(logits)
    dx_router, _, _ = O.router_backward(x_s, to_np(w_router), lg[tok], idx_np[tok], ds, "sigmoid", False, 1.0)
    assert_close(to_np(xg.grad[tt]), dx_routed + sh["dx"] + dx_router, TOL, "dX (sampled tokens)")

    announce("C3 full size: router weight gradient")
    # dW_r over every token, from the GPU's d(top_scores) (checked on the samples above)
    _, dwr, _ = O.router_backward(to_np(x), to_np(w_router), lg, idx_np, to_np(sc.grad), "sigmoid", False, 1.0)
    assert_close(to_np(wr.grad), dwr, TOL, "router dW")

    announce("C3 full size: shared expert weight gradients")
    gr = _spread(H, 32, rng)
    dc = _spread(H, 32, rng)
    xa, da_ = to_np(x), to_np(dout)
    g13, u13, c2 = O.expert_weight_grad_slices(xa, da_, sw13_np, sw2_np, gr, dc)
    assert_close(to_np(sw13.grad[torch.from_numpy(gr).to(DEV)]), g13, TOL, "shared dW13 gate rows")
    assert_close(to_np(sw13.grad[torch.from_numpy(H + gr).to(DEV)]), u13, TOL, "shared dW13 up rows")
    assert_close(to_np(sw2.grad[:, torch.from_numpy(dc).to(DEV)]).T, c2.T, TOL, "shared dW2 columns")
