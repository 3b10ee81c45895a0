"""Seeded random sweep of the fp8 e4m3 path over the options the fixed fp8
cases pin one at a time: expert counts from 1 to 19 with empty experts,
ragged row counts, model / hidden sizes from the smallest the block scales
allow upward, each of the three GEMM epilogues (plain store, clamp +
SwiGLU, score x un-permute scatter), the clamp on or off, and the whole
expert stage with top-k from 1 to 4 and the score before or after.

The GEMMs read the same e4m3 codes and fp32 block scales as the oracle,
whose semantics are "dequantise, fp32 GEMM": 1e-2 per row and norm-wise for
the GEMM units (bf16 output rounding plus fp32 summation order; the SwiGLU
activation to 1e-2 from the kernel's own bf16 h and to the path's bf16 bar
of 2e-2 from the oracle's), 5e-2, the fp8 tolerance of the path, for the
layer.  Each case names its seed and
shape before it runs."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, f32_dev, rand_bf16, to_np, topk_labels
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL_GEMM = 1e-2
TOL_LAYER = 5e-2


def _offs(counts):
    return torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(DEV)


def _quantised(rng, M, E, N, K):
    x = rand_bf16(rng, (M, K))
    w = rand_bf16(rng, (E, N, K), 0.02)
    xq, sx = O.quantize_fp8_rows(x)
    wq, sw = O.quantize_fp8_blocks(w)
    dev = [torch.from_numpy(xq).to(DEV), f32_dev(np.ascontiguousarray(sx.T)), torch.from_numpy(wq).to(DEV), f32_dev(sw)]
    return xq, sx, wq, sw, dev


@pytest.mark.parametrize("seed", range(15))
def test_sweep_fp8_gemms_vs_oracle(ops, seed):
    rng = np.random.default_rng(9100 + seed)
    E = int(rng.integers(1, 20))
    counts = rng.integers(0, 400, E) * (rng.random(E) > 0.15)
    if counts.sum() == 0:
        counts[0] = 7
    M = int(counts.sum())
    D = int(rng.choice([128, 256, 384, 512]))
    H = int(rng.choice([128, 192, 256, 320]))  # the SwiGLU kernel takes H % 64 == 0
    epi = ["store", "swiglu", "scatter"][seed % 3]
    limit = [None, 0.5][(seed // 3) % 2]
    offs = np.cumsum(counts)
    announce(f"fp8 sweep seed={seed} {epi} counts={counts.tolist()} D={D} H={H} limit={limit}")
    if epi == "swiglu":
        xq, sx, wq, sw, d = _quantised(rng, M, E, 2 * H, D)
        a, h = ops.grouped_mm_fp8_swiglu(*d, _offs(counts), limit, save_h=True)
        href = O.bf16_round(O.grouped_mm_fp8(xq, sx, wq, sw, offs))
        assert_close(to_np(h), href, TOL_GEMM, "h")
        # the activation is computed from the bf16 pre-activation the kernel
        # stored; against the oracle's own h a one-ulp bf16 difference of h
        # (summation order) carries through silu(gate) * up, so that
        # comparison takes the path's bf16 bar, as the bf16 GEMM tests do
        assert_close(to_np(a), O.swiglu(to_np(h), limit), TOL_GEMM, "a from the kernel's h")
        assert_close(to_np(a), O.swiglu(href, limit), 2e-2, "a")
    elif epi == "store":
        xq, sx, wq, sw, d = _quantised(rng, M, E, 2 * H, D)
        out = ops.grouped_mm_fp8(*d, _offs(counts))
        assert_close(to_np(out), O.grouped_mm_fp8(xq, sx, wq, sw, offs), TOL_GEMM, "store")
    else:
        K = 128 * ((H + 127) // 128)  # w2's reduction: whole 128-channel scale blocks
        xq, sx, wq, sw, d = _quantised(rng, M, E, D, K)
        dest = rng.permutation(M).astype(np.int32)
        scale = rng.random(M).astype(np.float32)
        out = ops.grouped_mm_fp8_unpermute(*d, _offs(counts), f32_dev(scale), torch.from_numpy(dest).to(DEV), M)
        y = O.grouped_mm_fp8(xq, sx, wq, sw, offs) * scale[:, None]
        ref = np.zeros_like(y)
        ref[dest] = y
        assert_close(to_np(out), ref, TOL_GEMM, "scatter")


@pytest.mark.parametrize("seed", range(6))
def test_sweep_fp8_layer_vs_oracle(pkg, ops, seed):
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(9300 + seed)
    E = int(rng.integers(2, 17))
    K = int(rng.integers(1, min(E, 4) + 1))
    T = int(rng.integers(16, 500))
    D = int(rng.choice([128, 256, 512]))
    H = int(rng.choice([128, 256, 384]))  # w2 reads a in whole 128-channel scale blocks
    before = bool(rng.integers(0, 2))
    limit = [None, 0.5][int(rng.integers(0, 2))]
    x = rand_bf16(rng, (T, D))
    w13 = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2 = rand_bf16(rng, (E, D, H), 0.02)
    idx = topk_labels(T, K, E, rng)
    scores = (rng.random((T, K)) * 0.8 + 0.2).astype(np.float32)
    announce(f"fp8 layer sweep seed={seed} T={T} D={D} H={H} E={E} K={K} before={before} limit={limit}")
    w13q, s13 = ops.quantize_fp8_blocks(bf16_dev(w13))
    w2q, s2 = ops.quantize_fp8_blocks(bf16_dev(w2))
    out = F.moe_experts_forward_fp8(bf16_dev(x), f32_dev(scores), torch.from_numpy(idx).to(DEV), w13q, s13,
                                    w2q, s2, E, before, limit)
    b13, c13 = O.quantize_fp8_blocks(w13)
    b2, c2 = O.quantize_fp8_blocks(w2)
    ref = O.moe_forward_fp8(x, scores, idx, b13, c13, b2, c2, E, before, limit)
    assert out.shape == (T, D)
    assert_close(to_np(out), ref, TOL_LAYER, f"fp8 layer sweep seed {seed}")
