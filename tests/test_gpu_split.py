"""GPU parity of the forward / dgrad grouped GEMMs' tail split.

The persistent walk runs R full rounds of one tile per workgroup; the rt
tiles left over are cut along k into np pieces that run on the idle
workgroups, and the last piece of a tile to arrive adds every piece's fp32
partial sums in piece order before the epilogue.  Each case below is sized
so that its leftover tiles are split on the device at hand (asserted from
the device's CU count), and is checked against the oracle per row, for
bit-identical results over repeated calls (the sum order does not depend
on which piece arrives last), and, through the C-ABI, for the plan's
arrival counters being back at zero afterwards.  Tolerance as the other
GEMM tests: max relative error 2e-2, norm-wise and per row.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, f32_dev, rand_bf16, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2
TQ = 320  # token rows per tile: counts of 320 or fewer rows give one tile each


def _grid() -> int:
    return (torch.cuda.get_device_properties(0).multi_processor_count + 7) & ~7


def _pieces(ntiles: int, ksteps: int) -> int:
    """Pieces per leftover tile: at most 8, G // rt, ksteps // 8 and
    sqrt(ksteps / 2), two only for 64 stages or more, none after more than
    6 full rounds (the kernel's rule)."""
    G = _grid()
    rt = ntiles % G
    if rt == 0 or rt > 512 or ntiles // G > 6:
        return 1
    n = max(1, min(G // rt, 8, ksteps // 8))
    while n > 1 and ksteps < 2 * n * n:
        n -= 1
    return 1 if n == 2 and ksteps < 64 else n


def _qtiles(counts) -> int:
    return sum(-(-int(c) // TQ) for c in counts)


def _offs(counts):
    return torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(DEV)


def _expect_split(counts, n_wtiles: int, kred: int) -> None:
    ntiles = _qtiles(counts) * n_wtiles
    n = _pieces(ntiles, kred // 64)
    assert n > 1, f"case does not split on this device ({ntiles} tiles, {kred // 64} k stages, grid {_grid()})"


def _repeat_identical(fn, n=2):
    first = fn()
    for _ in range(n):
        again = fn()
        for a, b in zip(first if isinstance(first, tuple) else (first,), again if isinstance(again, tuple) else (again,)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "split sum differs between calls"
    return first


# counts: every expert's rows fit one tile except where stated
COUNTS = (320, 320, 200)


@pytest.mark.parametrize("counts,N,K", [(COUNTS, 2048, 4096),          # 24 tiles, 64 stages: 5 pieces
                                        ((320,) * 35, 2048, 1600)])   # 280 tiles: one full round + 24, 3 pieces
def test_split_grouped_mm(ops, counts, N, K):
    counts = np.array(counts, np.int64)
    M, E = int(counts.sum()), len(counts)
    _expect_split(counts, N // 256, K)
    rng = np.random.default_rng(M + N + K)
    x, w = rand_bf16(rng, (M, K)), rand_bf16(rng, (E, N, K), 0.05)
    announce(f"split grouped_mm M={M} E={E} N={N} K={K}")
    xd, wd, od = bf16_dev(x), bf16_dev(w), _offs(counts)
    out = _repeat_identical(lambda: ops.grouped_mm(xd, wd, od))
    assert_close(to_np(out), O.grouped_mm(x, w, np.cumsum(counts)), TOL, "out")


def test_split_counters_back_at_zero(ops):
    counts = np.array(COUNTS, np.int64)
    M, E, N, K = int(counts.sum()), len(counts), 2048, 4096
    _expect_split(counts, N // 256, K)
    rng = np.random.default_rng(5)
    x, w = bf16_dev(rand_bf16(rng, (M, K))), bf16_dev(rand_bf16(rng, (E, N, K), 0.05))
    lib = ops._lib.load()
    wsb = int(lib.ttamd_gemm_workspace_bytes(M, E))
    plan_b = int(lib.ttamd_gemm_plan_bytes(M, E))
    assert wsb >= plan_b + _grid() * 327680
    ws = torch.full((wsb,), 0x7F, dtype=torch.uint8, device=DEV)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    announce("split counters")
    ops._lib.call("ttamd_grouped_mm", ops._p(x), ops._p(w), ops._p(_offs(counts)), M, E, N, K, ops._p(out),
                  ops._p(ws), wsb, ops._stream(DEV))
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    assert not raw[16 : 16 + 4 * 512].any(), "split-tile arrival counters must be back at zero"
    ref = O.grouped_mm(to_np(x), to_np(w), np.cumsum(counts))
    assert_close(to_np(out), ref, TOL, "out")


@pytest.mark.parametrize("limit", [None, 0.75])
def test_split_swiglu(ops, limit):
    counts = np.array(COUNTS, np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 4096, 1024
    _expect_split(counts, H // 128, D)
    rng = np.random.default_rng(11)
    x, w13 = rand_bf16(rng, (M, D)), rand_bf16(rng, (E, 2 * H, D), 0.05)
    announce(f"split swiglu limit={limit}")
    xd, wd, od = bf16_dev(x), bf16_dev(w13), _offs(counts)
    a, h = _repeat_identical(lambda: ops.grouped_mm_swiglu(xd, wd, od, limit, save_h=True))
    h_ref = O.bf16_round(O.grouped_mm(x, w13, np.cumsum(counts)))
    assert_close(to_np(h), h_ref, TOL, "h")
    assert_close(to_np(a), O.swiglu(h_ref, limit), TOL, "a")


def test_split_swiglu_gather(ops):
    counts = np.array(COUNTS, np.int64)
    K = 2
    M, E, D, H = int(counts.sum()), len(counts), 2048, 1024
    T = M // K
    _expect_split(counts, H // 128, D)
    rng = np.random.default_rng(12)
    labels = rng.permutation(np.repeat(np.arange(E), counts))
    sidx = O.stable_order(labels, E).astype(np.int32)
    x, w13 = rand_bf16(rng, (T, D)), rand_bf16(rng, (E, 2 * H, D), 0.05)
    announce("split swiglu gather")
    xd, sd, wd, od = bf16_dev(x), torch.from_numpy(sidx).to(DEV), bf16_dev(w13), _offs(counts)
    a, h = _repeat_identical(lambda: ops.grouped_mm_swiglu_gather(xd, sd, K, wd, od, None, save_h=True))
    h_ref = O.bf16_round(O.grouped_mm(x[sidx // K], w13, np.cumsum(counts)))
    assert_close(to_np(h), h_ref, TOL, "h")
    assert_close(to_np(a), O.swiglu(h_ref), TOL, "a")


def test_split_unpermute_scatter(ops):
    counts = np.array(COUNTS, np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 2048, 2048
    _expect_split(counts, D // 256, H)
    rng = np.random.default_rng(13)
    a, w2 = rand_bf16(rng, (M, H)), rand_bf16(rng, (E, D, H), 0.05)
    dest = rng.permutation(M).astype(np.int32)
    scale = rng.random(M).astype(np.float32)
    announce("split unpermute scatter")
    ad, wd, od, sd, dd = bf16_dev(a), bf16_dev(w2), _offs(counts), f32_dev(scale), torch.from_numpy(dest).to(DEV)
    out = _repeat_identical(lambda: ops.grouped_mm_unpermute(ad, wd, od, sd, dd, M))
    ref = np.zeros((M, D), np.float32)
    ref[dest] = O.grouped_mm(a, w2, np.cumsum(counts)) * scale[:, None]
    assert_close(to_np(out), ref, TOL, "out")


def _dgrad_ref(dy, w, counts):
    offs = np.cumsum(counts)
    ref = np.zeros((dy.shape[0], w.shape[2]), np.float32)
    s = 0
    for e, t in enumerate(offs):
        ref[s:t] = dy[s:t] @ w[e]
        s = t
    return ref


def test_split_dgrad(ops):
    counts = np.array(COUNTS, np.int64)
    M, E, N, K = int(counts.sum()), len(counts), 4096, 1024
    _expect_split(counts, K // 256, N)
    rng = np.random.default_rng(14)
    dy, w = rand_bf16(rng, (M, N)), rand_bf16(rng, (E, N, K), 0.05)
    announce("split dgrad")
    dyd, wd, od = bf16_dev(dy), bf16_dev(w), _offs(counts)
    dx = _repeat_identical(lambda: ops.grouped_mm_dgrad(dyd, wd, od))
    assert_close(to_np(dx), _dgrad_ref(dy, w, counts), TOL, "dx")


def test_split_dgrad_swiglu(ops):
    counts = np.array(COUNTS, np.int64)
    M, E, D, H = int(counts.sum()), len(counts), 2048, 1024
    _expect_split(counts, H // 256, D)
    rng = np.random.default_rng(15)
    dy, w2, h = rand_bf16(rng, (M, D)), rand_bf16(rng, (E, D, H), 0.05), rand_bf16(rng, (M, 2 * H))
    announce("split dgrad swiglu")
    dyd, wd, hd, od = bf16_dev(dy), bf16_dev(w2), bf16_dev(h), _offs(counts)
    dh, a = _repeat_identical(lambda: ops.grouped_mm_dgrad_swiglu(dyd, wd, hd, od, None, want_a=True))
    g = _dgrad_ref(dy, w2, counts)
    gate, up = h[:, :H].astype(np.float64), h[:, H:].astype(np.float64)
    sig = 1 / (1 + np.exp(-gate))
    ref = np.concatenate([g * up * sig * (1 + gate * (1 - sig)), g * gate * sig], axis=1)
    assert_close(to_np(dh)[:, :H], ref[:, :H], TOL, "dgate")
    assert_close(to_np(dh)[:, H:], ref[:, H:], TOL, "dup")
    assert_close(to_np(a), O.swiglu(h), 1e-2, "a")
