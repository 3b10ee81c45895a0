"""Pins the oracle's floating-point functions (CPU only).

Checks: torch._grouped_mm bf16 chain (the reference's own op sequence,
npu_gmm.py:29-38), torch autograd of an fp32 restatement (index_add form of
qwen3_5/model.py:703-735), torch softmax/sigmoid/topk, torch bf16 casts,
and planted mistakes that the checks must catch.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_names, load_golden
from oracle import moe_oracle as O


def _limit(g):
    v = float(g["limit"])
    return None if np.isnan(v) else v


def test_bf16_round_matches_torch():
    g = load_golden("bf16_round")
    np.testing.assert_array_equal(O.bf16_round(g["values"]), g["rounded"])


@pytest.mark.parametrize("name", golden_names("experts_"))
def test_experts_forward_matches_torch_grouped_mm(name):
    g = load_golden(name)
    y, h, a = O.experts_forward(g["x"], g["w13"], g["w2"], g["counts"], _limit(g), round_intermediates=True)
    M = int(g["counts"].sum())
    # h: same products, same rounding point; accumulation order may differ by an ulp
    assert O.max_rel_err(h[:M], O.bf16_round(g["h_f32"])) < 1e-2
    L = _limit(g)
    if L is not None:  # the reference keeps the clamped h (npu_gmm.py:33-36)
        H = h.shape[1] // 2
        hc = np.concatenate([np.minimum(h[:, :H], L), np.clip(h[:, H:], -L, L)], axis=1)
        assert O.max_rel_err(hc[:M], g["h_bf16"]) < 1e-2
    assert O.max_rel_err(a[:M], g["a_bf16"]) < 2e-2
    assert O.max_rel_err(y[:M], g["y_bf16"]) < 2e-2
    # the unclamped pre-activation agrees with the fp32 per-expert loop
    yf, hf, _ = O.experts_forward(g["x"], g["w13"], g["w2"], g["counts"], None, round_intermediates=False)
    assert O.max_rel_err(hf[:M], g["h_f32"]) < 1e-5


@pytest.mark.parametrize("name", golden_names("layer_"))
def test_moe_forward_matches_autograd_golden(name):
    g = load_golden(name)
    E = int(g["num_experts"])
    out = O.moe_forward(g["x"], g["scores"], g["idx"], g["w13"], g["w2"], E, bool(g["score_before"]),
                        _limit(g), round_intermediates=False)
    assert O.max_rel_err(out, g["out"]) < 1e-5


@pytest.mark.parametrize("name", golden_names("layer_"))
def test_moe_backward_matches_autograd_golden(name):
    g = load_golden(name)
    E = int(g["num_experts"])
    grads = O.moe_backward(g["x"], g["scores"], g["idx"], g["w13"], g["w2"], E, bool(g["score_before"]),
                           g["dout"], _limit(g))
    for k in ("dx", "dw13", "dw2", "dscores"):
        assert O.max_rel_err(grads[k], g[k]) < 1e-4, k


@pytest.mark.parametrize("name", golden_names("layer_"))
def test_moe_backward_bf16_intermediates_near_golden(name):
    """Rounding the forward intermediates to bf16 (as the reference stores
    them) moves the gradients by no more than bf16 noise."""
    g = load_golden(name)
    E = int(g["num_experts"])
    grads = O.moe_backward(g["x"], g["scores"], g["idx"], g["w13"], g["w2"], E, bool(g["score_before"]),
                           g["dout"], _limit(g), round_intermediates=True)
    for k in ("dx", "dw13", "dw2", "dscores"):
        assert O.max_rel_err(grads[k], g[k]) < 2e-2, k


def test_moe_forward_brute_token_loop():
    """Per-token loop in the form of qwen3_5/model.py:703-735 (weights applied
    after the expert, summed with index_add) for the score-after layout."""
    rng = np.random.default_rng(11)
    T, K, E, D, H = 10, 2, 5, 16, 8
    x = rng.standard_normal((T, D)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * H, D)) * 0.3).astype(np.float32)
    w2 = (rng.standard_normal((E, D, H)) * 0.3).astype(np.float32)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    sc = rng.random((T, K)).astype(np.float32)
    ref = np.zeros((T, D))
    for t in range(T):
        for k in range(K):
            e = idx[t, k]
            h = w13[e].astype(np.float64) @ x[t]
            a = h[:H] / (1 + np.exp(-h[:H])) * h[H:]
            ref[t] += sc[t, k] * (w2[e].astype(np.float64) @ a)
    out = O.moe_forward(x, sc, idx, w13, w2, E, False, None, round_intermediates=False)
    assert O.max_rel_err(out, ref) < 1e-5


def test_finite_difference_dscores():
    """Central differences of the fp64-evaluated forward w.r.t. one score."""
    rng = np.random.default_rng(12)
    T, K, E, D, H = 6, 2, 3, 8, 4
    x = rng.standard_normal((T, D)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * H, D)) * 0.5).astype(np.float32)
    w2 = (rng.standard_normal((E, D, H)) * 0.5).astype(np.float32)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    sc = (rng.random((T, K)) + 0.5).astype(np.float32)
    dout = rng.standard_normal((T, D)).astype(np.float32)
    for before in (False, True):
        grads = O.moe_backward(x, sc, idx, w13, w2, E, before, dout)
        for (t, k) in ((0, 0), (3, 1)):
            eps = 1e-2
            sp, sm = sc.copy(), sc.copy()
            sp[t, k] += eps
            sm[t, k] -= eps
            fp = O.moe_forward(x, sp, idx, w13, w2, E, before, None, round_intermediates=False)
            fm = O.moe_forward(x, sm, idx, w13, w2, E, before, None, round_intermediates=False)
            fd = ((fp.astype(np.float64) - fm) * dout).sum() / (2 * eps)
            assert abs(fd - grads["dscores"][t, k]) < 2e-3 * max(1.0, abs(fd)), (before, t, k)


@pytest.mark.parametrize("name", golden_names("router_"))
def test_router_topk_matches_torch(name):
    g = load_golden(name)
    func = "softmax" if "softmax" in name else "sigmoid"
    norm = name.endswith("norm")
    K = int(g["top_k"])
    s, i = O.router_topk(g["logits"], K, func, norm)
    np.testing.assert_array_equal(i, g["indices"])
    np.testing.assert_allclose(s, g["scores"], rtol=1e-6, atol=1e-7)
    s, i = O.router_topk(g["logits"], K, func, False, expert_bias=g["bias"])
    np.testing.assert_array_equal(i, g["indices_bias"])
    np.testing.assert_allclose(s, g["scores_bias"], rtol=1e-6, atol=1e-7)


def _bf16_ulp(v):
    """Spacing of bf16 values at |v| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 1e-30)))
    return np.exp2(e - 7)


def test_router_logits_match_torch_linear():
    """F.linear in fp32 rounded to bf16 (torch golden): exact bf16 values up to
    one bf16 step on a few entries (summation order); a missing bf16
    rounding or a transposed weight fails it."""
    g = load_golden("gate_linear")
    z = O.router_logits(g["x"], g["w"])
    d = np.abs(z - g["logits"])
    assert np.all(d <= _bf16_ulp(g["logits"]) * 1.01)
    assert (d > 0).mean() < 0.01
    unrounded = (np.asarray(g["x"], np.float64) @ np.asarray(g["w"], np.float64).T).astype(np.float32)
    assert (unrounded != g["logits"]).mean() > 0.5
    with pytest.raises(ValueError):
        O.router_logits(g["x"], g["w"].T)


def test_shared_expert_add_matches_torch_block():
    """The reference block's shared-expert tail in torch bf16 (golden):
    gated and ungated within one bf16 step; dropping the gate fails it."""
    g = load_golden("shared_expert_gated")
    out = O.shared_expert_add(g["routed"], g["x"], g["w13"], g["w2"], g["gate_logits"])
    assert O.max_rel_err(out, g["out"]) < 1e-2
    out0 = O.shared_expert_add(g["routed"], g["x"], g["w13"], g["w2"], None)
    assert O.max_rel_err(out0, g["out_ungated"]) < 1e-2
    assert O.max_rel_err(out0, g["out"]) > 5e-2


def test_router_ties_prefer_lower_expert():
    logits = np.array([[1.0, 3.0, 3.0, 0.0, 3.0], [2.0, 2.0, 2.0, 2.0, 2.0]], np.float32)
    _, i = O.router_topk(logits, 3, "sigmoid")
    np.testing.assert_array_equal(i, [[1, 2, 4], [0, 1, 2]])


def test_planted_gate_up_swap_is_caught():
    """Swapping gate and up halves (a plausible layout mistake) fails the golden."""
    g = load_golden("experts_nolimit")
    H = g["w13"].shape[1] // 2
    w13_swapped = np.concatenate([g["w13"][:, H:], g["w13"][:, :H]], axis=1)
    y, _, _ = O.experts_forward(g["x"], w13_swapped, g["w2"], g["counts"], None)
    assert O.max_rel_err(y, g["y_bf16"]) > 0.1


def test_planted_missing_score_is_caught():
    g = load_golden("layer_k2_after")
    out = O.moe_forward(g["x"], np.ones_like(g["scores"]), g["idx"], g["w13"], g["w2"], int(g["num_experts"]),
                        False, None, round_intermediates=False)
    assert O.max_rel_err(out, g["out"]) > 0.1


@pytest.mark.parametrize("limit", [None, 0.3])
def test_expert_weight_grad_slices_match_full_backward(limit):
    """The slice form equals the matching rows / columns of moe_backward's
    full per-expert gradients (a swapped gate/up half, a transposed slice or
    a dropped clamp mask fails it)."""
    rng = np.random.default_rng(21)
    T, E, D, H = 40, 3, 16, 12
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w13 = O.bf16_round((rng.standard_normal((E, 2 * H, D)) * 0.4).astype(np.float32))
    w2 = O.bf16_round((rng.standard_normal((E, D, H)) * 0.4).astype(np.float32))
    idx = rng.integers(0, E, (T, 1))
    sc = (rng.random((T, 1)) * 0.8 + 0.2).astype(np.float32)
    dout = rng.standard_normal((T, D)).astype(np.float32)
    for before in (True, False):
        full = O.moe_backward(x, sc, idx, w13, w2, E, before, dout, limit, round_intermediates=True)
        for e in range(E):
            rows = np.nonzero(idx[:, 0] == e)[0]  # stable order of one expert's tokens
            routed = x[rows]
            if before:
                routed = O.bf16_round(routed * sc[rows])
                dy = dout[rows]
            else:
                dy = dout[rows] * sc[rows]
            gr, dc = np.array([0, 5, H - 1]), np.array([1, H - 2])
            g13, u13, c2 = O.expert_weight_grad_slices(routed, dy, w13[e], w2[e], gr, dc, limit)
            np.testing.assert_allclose(g13, full["dw13"][e][gr], rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(u13, full["dw13"][e][H + gr], rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(c2, full["dw2"][e][:, dc], rtol=1e-5, atol=1e-6)


def test_swiglu_backward_finite_differences():
    rng = np.random.default_rng(22)
    H, L = 6, 0.7
    h = (rng.standard_normal((5, 2 * H)) * 1.5).astype(np.float64)
    da = rng.standard_normal((5, H))
    for limit in (None, L):
        dh = O.swiglu_backward(da.astype(np.float32), h.astype(np.float32), limit).astype(np.float64)
        eps = 1e-4

        def f(hh):
            gate, up = hh[:, :H], hh[:, H:]
            if limit is not None:
                up, gate = np.clip(up, -limit, limit), np.minimum(gate, limit)
            return (gate / (1 + np.exp(-gate)) * up * da).sum()
        for (r, c) in ((0, 0), (2, 3), (4, H + 1), (1, H + 5)):
            if limit is not None and abs(abs(h[r, c]) - limit) < 1e-3:
                continue  # at the kink
            hp, hm = h.copy(), h.copy()
            hp[r, c] += eps
            hm[r, c] -= eps
            fd = (f(hp) - f(hm)) / (2 * eps)
            assert abs(fd - dh[r, c]) < 1e-3 * max(1.0, abs(fd)), (limit, r, c)


def test_swiglu_clamp_special_values_match_torch_autograd():
    """NaN, +-inf, values on the limit and signed zeros through the
    reference's op sequence (npu_gmm.py:32-37: torch.clamp of up and gate,
    then silu(gate) * up) under torch autograd on the CPU, against the
    oracle's forward and backward: torch.clamp keeps NaN in its forward and
    its backward is where(in range, grad, 0)."""
    import math

    import torch
    import torch.nn.functional as F

    L = 0.5
    vals = [math.nan, math.inf, -math.inf, L, -L, 0.0, -0.0, 0.3, -0.3, 2.0, -2.0]
    pairs = [(g, u) for g in vals for u in vals]
    h = np.array(pairs, np.float32)  # [n, 2]: H = 1, gate then up
    da = np.random.default_rng(24).standard_normal((len(pairs), 1)).astype(np.float32)

    hh = torch.tensor(h, requires_grad=True)
    gate, up = hh.chunk(2, -1)
    up = torch.clamp(up, min=-L, max=L)
    gate = torch.clamp(gate, max=L)
    a = F.silu(gate) * up
    a.backward(torch.tensor(da))
    want_a = a.detach().numpy()
    want_dh = hh.grad.numpy()

    got_a = O.swiglu(h, L)
    got_dh = O.swiglu_backward(da, h, L)
    for got, want, what in ((got_a, want_a, "forward"), (got_dh, want_dh, "backward")):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want), err_msg=f"{what}: NaN positions")
        fin = ~np.isnan(want)
        np.testing.assert_allclose(got[fin], want[fin], rtol=1e-6, atol=1e-7, err_msg=what)
    # the clamp's gradient is exactly zero where it clamps or meets NaN
    g_out = (h[:, 0] > L) | np.isnan(h[:, 0])
    u_out = (np.abs(h[:, 1]) > L) | np.isnan(h[:, 1])
    assert (got_dh[g_out, 0] == 0).all() and (got_dh[u_out, 1] == 0).all()


def test_dscores_abs_bounds_dscores():
    """The dot-product scale returned with dscores bounds it: |<a,b>| <= sum|a b|."""
    rng = np.random.default_rng(23)
    T, K, E, D, H = 30, 2, 4, 16, 8
    x = rng.standard_normal((T, D)).astype(np.float32)
    w13 = (rng.standard_normal((E, 2 * H, D)) * 0.3).astype(np.float32)
    w2 = (rng.standard_normal((E, D, H)) * 0.3).astype(np.float32)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    sc = rng.random((T, K)).astype(np.float32)
    dout = rng.standard_normal((T, D)).astype(np.float32)
    for before in (True, False):
        g = O.moe_backward(x, sc, idx, w13, w2, E, before, dout)
        assert (np.abs(g["dscores"]) <= g["dscores_abs"] * (1 + 1e-5)).all()
        assert (g["dscores_abs"] > 0).all()


def test_grouped_dgrad_wgrad_brute_force():
    rng = np.random.default_rng(24)
    M, E, N, K = 9, 4, 5, 3
    counts = np.array([3, 0, 4, 1])  # one empty expert, one row past the last offset
    offs = np.cumsum(counts)
    dy = rng.standard_normal((M, N)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((E, N, K)).astype(np.float32)
    dx = O.grouped_dgrad(dy, w, offs)
    dw = O.grouped_wgrad(dy, x, offs, E)
    e_of = np.searchsorted(offs, np.arange(M), side="right")
    for m in range(M):
        for k in range(K):
            want = sum(float(dy[m, n]) * float(w[e_of[m], n, k]) for n in range(N)) if m < offs[-1] else 0.0
            assert abs(dx[m, k] - want) < 1e-5
    for e in range(E):
        for n in range(N):
            for k in range(K):
                want = sum(float(dy[m, n]) * float(x[m, k]) for m in range(M) if m < offs[-1] and e_of[m] == e)
                assert abs(dw[e, n, k] - want) < 1e-5
    assert not dw[1].any()
