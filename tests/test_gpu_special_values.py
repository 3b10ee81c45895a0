"""NaN and infinities through the clamp + SwiGLU epilogues, against the
oracle, which follows torch.clamp (npu_gmm.py:33-35): its forward keeps a
NaN (it does not turn it into the limit), and its backward is
where(in range, grad, 0), exactly zero where it clamped or met NaN.

* forward, bf16 and fp8 w13: token rows holding a NaN or an infinity give
  pre-activations h of NaN / +-inf; the activation must be NaN exactly where
  the oracle's is, +-inf with the same sign, and the finite rest within the
  GEMM tolerance per row;
* backward (dgrad fused with the SwiGLU backward): chosen columns of the
  saved h set to NaN, +-inf, +-L, values just past the limit and signed
  zeros, with and without the clamp."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, f32_dev, rand_bf16, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2


def assert_close_special(got, ref, tol, what):
    """NaN exactly where the reference is NaN, +-inf where it is +-inf (same
    sign), the finite rest within tol (norm-wise and per row)."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref), err_msg=f"{what}: NaN positions")
    inf = np.isinf(ref)
    np.testing.assert_array_equal(np.isinf(got), inf, err_msg=f"{what}: inf positions")
    np.testing.assert_array_equal(got[inf], ref[inf], err_msg=f"{what}: inf signs")
    fin = np.isfinite(ref)
    assert_close(np.where(fin, got, 0), np.where(fin, ref, 0), tol, what)


def _offs(counts):
    return torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(DEV)


@pytest.mark.parametrize("limit", [None, 0.5])
def test_swiglu_forward_nan_and_inf_rows(ops, limit):
    rng = np.random.default_rng(4100)
    counts = np.array([150, 0, 200, 90], np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 256, 192
    x = rand_bf16(rng, (M, D))
    x[5, :] = np.nan          # h row all NaN
    x[160, 7] = np.inf        # h row +-inf by the sign of w13[e][:, 7]
    x[300, 3] = -np.inf
    w13 = rand_bf16(rng, (E, 2 * H, D), 0.08)
    announce(f"swiglu special rows limit={limit}")
    a, h = ops.grouped_mm_swiglu(bf16_dev(x), bf16_dev(w13), _offs(counts), limit, save_h=True)
    with np.errstate(invalid="ignore"):
        h_ref = O.bf16_round(O.grouped_mm(x, w13, np.cumsum(counts)))
    a_ref = O.swiglu(h_ref, limit)
    for r in (5, 160, 300):
        assert not np.isfinite(h_ref[r]).all(), r
    assert_close_special(to_np(h), h_ref, TOL, "h")
    assert_close_special(to_np(a), a_ref, TOL, "a")


@pytest.mark.parametrize("limit", [None, 0.5])
def test_fp8_swiglu_forward_nan_row(ops, limit):
    """A NaN activation scale (one k block of one token row) makes that
    row's h NaN in the oracle's dequantise-then-GEMM; the kernel applies the
    scale to the block's partial sum, which gives the same NaN."""
    rng = np.random.default_rng(4200)
    counts = np.array([300, 212], np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 512, 256
    x = rand_bf16(rng, (M, D))
    w = rand_bf16(rng, (E, 2 * H, D), 0.02)
    xq, sx = O.quantize_fp8_rows(x)
    wq, sw = O.quantize_fp8_blocks(w)
    sx = sx.copy()
    sx[17, 2] = np.nan
    sx[400, 0] = np.nan
    announce(f"fp8 swiglu NaN scale rows limit={limit}")
    a, h = ops.grouped_mm_fp8_swiglu(torch.from_numpy(xq).to(DEV), f32_dev(np.ascontiguousarray(sx.T)),
                                     torch.from_numpy(wq).to(DEV), f32_dev(sw), _offs(counts), limit, save_h=True)
    with np.errstate(invalid="ignore"):
        h_ref = O.bf16_round(O.grouped_mm_fp8(xq, sx, wq, sw, np.cumsum(counts)))
    a_ref = O.swiglu(h_ref, limit)
    assert np.isnan(h_ref[17]).all() and np.isnan(h_ref[400]).all()
    assert_close_special(to_np(h), h_ref, 1e-2, "h")
    assert_close_special(to_np(a), a_ref, 1e-2, "a")


@pytest.mark.parametrize("limit", [None, 0.5])
def test_swiglu_backward_special_values(ops, limit):
    rng = np.random.default_rng(4300)
    counts = np.array([130, 70, 0, 56], np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 256, 256
    dy = rand_bf16(rng, (M, D))
    w2 = rand_bf16(rng, (E, D, H), 0.08)
    h = rand_bf16(rng, (M, 2 * H))
    L = 0.5 if limit is None else limit
    just_past = float(O.bf16_round(np.array([L * 1.01], np.float32))[0])
    specials = [math.nan, math.inf, -math.inf, L, -L, just_past, -just_past, 0.0, -0.0]
    # gate column c and up column H + c' get the specials, in every pairing
    # over the first rows of each expert; other columns keep random values
    for i, g in enumerate(specials):
        for k, u in enumerate(specials):
            r = (i * len(specials) + k) % M
            h[r, 3 + i] = g
            h[r, H + 3 + k] = u
            h[r, 40 + i] = g          # the same gate values against a random up
            h[r, H + 80 + k] = u      # and the same up values against a random gate
    announce(f"dgrad_swiglu special values limit={limit}")
    dh, a = ops.grouped_mm_dgrad_swiglu(bf16_dev(dy), bf16_dev(w2), bf16_dev(h), _offs(counts), limit, want_a=True)
    offs = np.cumsum(counts)
    ref = O.swiglu_backward(O.grouped_dgrad(dy, w2, offs), h, limit)
    with np.errstate(invalid="ignore"):
        a_ref = O.swiglu(h, limit)
    got = to_np(dh)
    assert_close_special(got[:, :H], ref[:, :H], TOL, "d(gate)")
    assert_close_special(got[:, H:], ref[:, H:], TOL, "d(up)")
    assert_close_special(to_np(a), a_ref, 1e-2, "a")
    if limit is not None:
        # torch.clamp's gradient is exactly zero where it clamps or meets NaN
        g_out = (h[:, :H] > limit) | np.isnan(h[:, :H])
        u_out = (np.abs(h[:, H:]) > limit) | np.isnan(h[:, H:])
        assert (got[:, :H][g_out] == 0).all() and (got[:, H:][u_out] == 0).all()
