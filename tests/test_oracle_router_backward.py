"""Pins oracle.router_backward (CPU): against torch autograd of the upstream
router op sequence (golden fixtures from tests/golden/make_golden.py) and
against central finite differences of the float64 router forward.
Reference: the router forward it differentiates is the closed form at
torchtitanturbo/models/qwen3_5/model.py:757-765 (UPSTREAM TokenChoiceTopKRouter)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_names, load_golden
from oracle import moe_oracle as O


def _cfg(name):
    func = "softmax" if "softmax" in name else "sigmoid"
    return func, name.endswith("norm")


@pytest.mark.parametrize("name", golden_names("backward_router_"))
def test_router_backward_matches_torch_autograd(name):
    g = load_golden(name)
    func, norm = _cfg(name)
    dx, dw, dlog = O.router_backward(g["x"], g["w"], g["logits"], g["idx"], g["grad_top"], func, norm,
                                     float(g["route_scale"]))
    ref = g["dlogits"]
    # bf16 logit gradients: torch and the oracle sum the softmax Jacobian in
    # different orders, so allow one bf16 step (2^-8 relative) per element,
    # plus fp32 noise relative to the row: with softmax + renorm the
    # non-picked entries are -<ds, s> s_e, and <ds, s> is exactly
    # sum(g s) eps / S^2 ~ 0, so both sides hold rounding noise there
    row = np.abs(ref).max(axis=1, keepdims=True)
    step = np.abs(ref) * 2.0 ** -8 + 1e-6 * row
    assert np.all(np.abs(dlog - ref) <= step), np.abs(dlog - ref).max()
    sig = np.abs(ref) > 1e-4 * row  # entries that are not cancellation noise
    assert (dlog[sig] == ref[sig]).mean() > 0.9
    # torch's bf16 matmuls round dx, dw to bf16; the oracle keeps fp32
    for got, want in ((dx, g["dx"]), (dw, g["dw"])):
        err = np.abs(got - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-30)
        assert err.max() < 1e-2, err.max()


def test_router_backward_planted_mistake_fails_golden():
    """Dropping the renormalisation's denominator term (a plausible slip)
    must be caught by the golden check above."""
    g = load_golden("backward_router_softmax_k4_norm")
    s = O.router_scores(g["logits"], "softmax").astype(np.float64)
    idx = g["idx"]
    gt = g["grad_top"].astype(np.float64)
    picked = np.take_along_axis(s, idx, axis=-1)
    S = picked.sum(-1, keepdims=True) + 1e-20
    ds = np.zeros_like(s)
    np.add.at(ds, (np.arange(s.shape[0])[:, None], idx), gt / S)  # missing -sum(g s)/S^2
    dz = (ds - (ds * s).sum(-1, keepdims=True)) * s
    wrong = O.bf16_round(dz.astype(np.float32))
    assert np.abs(wrong - g["dlogits"]).max() > 10 * 2.0 ** -8 * np.abs(g["dlogits"]).max()


@pytest.mark.parametrize("func,norm,scale", [("softmax", True, 1.0), ("softmax", False, 2.0),
                                             ("sigmoid", False, 1.0), ("sigmoid", True, 0.5)])
def test_router_backward_finite_differences(func, norm, scale):
    rng = np.random.default_rng(3)
    T, D, E, K = 5, 16, 7, 3
    x = rng.standard_normal((T, D))
    w = rng.standard_normal((E, D)) * 0.3
    idx = np.argsort(-rng.random((T, E)), axis=1)[:, :K]
    gt = rng.standard_normal((T, K))
    logits = (x @ w.T).astype(np.float32)
    # the smooth path: logits and everything after in float64, no rounding
    dx, dw, _ = O.router_backward(x, w, logits, idx, gt, func, norm, scale, round_bf16=False)

    def f(xx, ww):
        return float((O.router_forward_f64(xx, ww, idx, func, norm, scale) * gt).sum())

    h = 1e-6
    ndx = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        ndx[i] = (f(xp, w) - f(xm, w)) / (2 * h)
    ndw = np.zeros_like(w)
    for i in np.ndindex(w.shape):
        wp, wm = w.copy(), w.copy()
        wp[i] += h
        wm[i] -= h
        ndw[i] = (f(x, wp) - f(x, wm)) / (2 * h)
    # logits pass through fp32 in the oracle's score step: 1e-4 relative
    assert np.abs(dx - ndx).max() <= 1e-4 * np.abs(ndx).max() + 1e-7
    assert np.abs(dw - ndw).max() <= 1e-4 * np.abs(ndw).max() + 1e-7
