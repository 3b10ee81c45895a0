"""GPU parity of the fp8 e4m3 path against the CPU oracle.

Quantisation is byte work derived from floats: codes and scales must be
bit-exact.  The fp8 GEMMs read the same codes and scales as the oracle, whose
reference semantics are "dequantise, fp32 GEMM": max relative error
(max|got-ref| / max|ref|) <= 1e-2 for the GEMM units (bf16 output rounding
plus fp32 summation order) and <= 5e-2, the fp8 tolerance the path is
specified to, for the layer."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, assert_close, bf16_dev, f32_dev, labels_from_counts, rand_bf16, to_np, zipf_counts
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
TOL_GEMM = 1e-2
TOL_LAYER = 5e-2


def _counts(kind, M, E, rng):
    if kind == "random":
        cut = np.sort(rng.integers(0, M + 1, E - 1))
        return np.diff(np.concatenate([[0], cut, [M]]))
    if kind == "zipf":
        return zipf_counts(M, E, 1.2, max(1, E - max(1, E // 8)), rng)
    raise ValueError(kind)


def _offs(counts):
    return torch.from_numpy(np.cumsum(counts).astype(np.int32)).to(DEV)


def _wide_range_bf16(rng, shape):
    """bf16 values with per-row magnitudes over six decades and one zero block."""
    x = rng.standard_normal(shape) * 10.0 ** rng.integers(-3, 3, (shape[0], 1))
    x[min(1, shape[0] - 1), :128] = 0.0
    return O.bf16_round(x.astype(np.float32))


@pytest.mark.parametrize("R,K", [(1, 128), (37, 384), (1000, 2048), (130, 7168)])
def test_quantize_rows_bit_exact(ops, R, K):
    rng = np.random.default_rng(R + K)
    x = _wide_range_bf16(rng, (R, K))
    announce(f"quantize_fp8_rows R={R} K={K}")
    q, s_t = ops.quantize_fp8_rows(bf16_dev(x))
    bits, scale = O.quantize_fp8_rows(x)
    np.testing.assert_array_equal(q.cpu().numpy(), bits)
    np.testing.assert_array_equal(s_t.cpu().numpy(), scale.T)


def test_quantize_rows_every_bf16_pattern(ops):
    """Every bf16 value of magnitude below 448 (both signs, subnormals, zero)
    through the row quantiser with a block scale of exactly 1 (each
    128-channel block also holds 448): the device e4m3 cast must equal the
    oracle's round-to-nearest-even cast on all of them."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) < 448.0)]
    nblk = (vals.size + 126) // 127
    x = np.zeros((nblk, 128), np.float32)
    x[:, 0] = 448.0
    flat = x[:, 1:].reshape(-1)
    flat[: vals.size] = vals
    x[:, 1:] = flat.reshape(nblk, 127)
    x = x.reshape(-1, 1024) if nblk % 8 == 0 else np.pad(x, ((0, 8 - nblk % 8), (0, 0))).reshape(-1, 1024)
    x[:, ::128] = 448.0
    announce(f"quantize_fp8_rows every bf16 pattern ({vals.size} values)")
    q, s_t = ops.quantize_fp8_rows(bf16_dev(x))
    ref_bits, ref_scale = O.quantize_fp8_rows(x)
    assert np.all(ref_scale == 1.0)
    np.testing.assert_array_equal(s_t.cpu().numpy(), ref_scale.T)
    np.testing.assert_array_equal(q.cpu().numpy(), ref_bits)


def test_quantize_rows_many_near_ties(ops):
    """29 M normal values with scales that are not powers of two: about a
    hundred quotients land within two fp32 ulps of an e4m3 halfway point,
    where only the exact division decides the rounding."""
    rng = np.random.default_rng(11)
    x = rand_bf16(rng, (4096, 7168))
    announce("quantize_fp8_rows 4096 x 7168 near-tie sweep")
    q, s_t = ops.quantize_fp8_rows(bf16_dev(x))
    bits, scale = O.quantize_fp8_rows(x)
    np.testing.assert_array_equal(s_t.cpu().numpy(), scale.T)
    np.testing.assert_array_equal(q.cpu().numpy(), bits)


@pytest.mark.parametrize("with_scale", [False, True])
def test_quantize_rows_gather_bit_exact(ops, with_scale):
    """Fused permute: routed row j = x[src_index[j] // K] (times the routing
    score rounded to bf16 when the score is applied before the experts)."""
    rng = np.random.default_rng(5 + with_scale)
    T, K, Dm = 300, 4, 512
    x = _wide_range_bf16(rng, (T, Dm))
    src = rng.permutation(T * K).astype(np.int32)
    mul = rng.random(T * K).astype(np.float32) if with_scale else None
    announce(f"quantize_fp8_rows gather scale={with_scale}")
    q, s_t = ops.quantize_fp8_rows(bf16_dev(x), torch.from_numpy(src).to(DEV), K,
                                   f32_dev(mul) if with_scale else None)
    rows = x[src // K]
    if with_scale:
        rows = O.bf16_round(rows * mul[:, None])
    bits, scale = O.quantize_fp8_rows(rows)
    np.testing.assert_array_equal(q.cpu().numpy(), bits)
    np.testing.assert_array_equal(s_t.cpu().numpy(), scale.T)


@pytest.mark.parametrize("E,N,K", [(1, 128, 128), (3, 256, 384), (2, 1024, 7168)])
def test_quantize_blocks_bit_exact(ops, E, N, K):
    rng = np.random.default_rng(E * N + K)
    w = rand_bf16(rng, (E, N, K), 0.02)
    w[0, :128, :128] = 0.0
    if E > 1:
        w[1, -128:, -128:] = O.bf16_round(w[1, -128:, -128:] * 1e-4)  # inputs stay bf16-exact
    announce(f"quantize_fp8_blocks E={E} N={N} K={K}")
    q, s = ops.quantize_fp8_blocks(bf16_dev(w))
    bits, scale = O.quantize_fp8_blocks(w)
    np.testing.assert_array_equal(s.cpu().numpy(), scale)
    np.testing.assert_array_equal(q.cpu().numpy(), bits)


def _quantised_operands(rng, M, E, N, K):
    x = rand_bf16(rng, (M, K))
    w = rand_bf16(rng, (E, N, K), 0.02)
    xq, sx = O.quantize_fp8_rows(x)
    wq, sw = O.quantize_fp8_blocks(w)
    dev = dict(
        xq=torch.from_numpy(xq).to(DEV), sx_t=f32_dev(np.ascontiguousarray(sx.T)),
        wq=torch.from_numpy(wq).to(DEV), sw=f32_dev(sw),
    )
    return xq, sx, wq, sw, dev


@pytest.mark.parametrize("M,E,N,K,kind", [(1000, 8, 256, 256, "random"), (700, 4, 512, 2048, "zipf"),
                                          (129, 3, 128, 128, "random"), (333, 32, 384, 512, "zipf")])
def test_grouped_mm_fp8(ops, M, E, N, K, kind):
    rng = np.random.default_rng(M + E + N + K)
    counts = _counts(kind, M, E, rng)
    xq, sx, wq, sw, d = _quantised_operands(rng, M, E, N, K)
    announce(f"grouped_mm_fp8 M={M} E={E} N={N} K={K} {kind}")
    out = ops.grouped_mm_fp8(d["xq"], d["sx_t"], d["wq"], d["sw"], _offs(counts))
    ref = O.grouped_mm_fp8(xq, sx, wq, sw, np.cumsum(counts))
    assert_close(to_np(out), ref, TOL_GEMM, "to_np(out)")


@pytest.mark.parametrize("limit", [None, 0.75])
@pytest.mark.parametrize("M,E,D,H,kind", [(1000, 8, 256, 128, "random"), (2048, 16, 512, 192, "zipf"),
                                          (300, 4, 2048, 768, "random")])
def test_grouped_mm_fp8_swiglu(ops, M, E, D, H, kind, limit):
    rng = np.random.default_rng(M + D + H)
    counts = _counts(kind, M, E, rng)
    xq, sx, wq, sw, d = _quantised_operands(rng, M, E, 2 * H, D)
    announce(f"grouped_mm_fp8_swiglu M={M} E={E} D={D} H={H} limit={limit}")
    a, h = ops.grouped_mm_fp8_swiglu(d["xq"], d["sx_t"], d["wq"], d["sw"], _offs(counts), limit, save_h=True)
    href = O.bf16_round(O.grouped_mm_fp8(xq, sx, wq, sw, np.cumsum(counts)))
    aref = O.swiglu(href, limit)
    assert_close(to_np(h), href, TOL_GEMM, "to_np(h)")
    assert_close(to_np(a), aref, TOL_GEMM, "to_np(a)")


@pytest.mark.parametrize("topk", [1, 4])
def test_grouped_mm_fp8_unpermute_scatter_scale(ops, topk):
    rng = np.random.default_rng(17 + topk)
    T, E, D, H = 256, 8, 256, 384
    M = T * topk
    counts = _counts("random", M, E, rng)
    aq, sa, wq, sw, d = _quantised_operands(rng, M, E, D, H)
    dest = rng.permutation(M).astype(np.int32)
    scale = rng.random(M).astype(np.float32)
    announce(f"grouped_mm_fp8_unpermute topk={topk}")
    out = ops.grouped_mm_fp8_unpermute(d["xq"], d["sx_t"], d["wq"], d["sw"], _offs(counts), f32_dev(scale),
                                       torch.from_numpy(dest).to(DEV), M)
    y = O.grouped_mm_fp8(aq, sa, wq, sw, np.cumsum(counts)) * scale[:, None]
    ref = np.zeros_like(y)
    ref[dest] = y
    assert_close(to_np(out), ref, TOL_GEMM, "to_np(out)")


# One expert per tile height that changes the k loop's per-wave token-block
# count (each wave computes 0, 2, 4, 6 or 8 blocks of 16 rows of its
# 128-row half of the 256-row tile and skips the rest), plus experts split
# into several tiles and one without rows.
TILE_HEIGHTS = np.array([1, 16, 17, 31, 32, 33, 48, 64, 65, 96, 97, 127, 128, 129, 144, 145, 160, 161,
                         192, 200, 224, 240, 255, 256, 0, 257, 300, 511, 513])


@pytest.mark.parametrize("epi", ["store", "swiglu", "scatter"])
def test_fp8_every_tile_height(ops, epi):
    rng = np.random.default_rng(91)
    counts = TILE_HEIGHTS
    E, M = counts.size, int(counts.sum())
    offs = _offs(counts)
    announce(f"fp8 tile heights epi={epi} M={M} E={E}")
    if epi == "store":
        xq, sx, wq, sw, d = _quantised_operands(rng, M, E, 384, 256)
        out = ops.grouped_mm_fp8(d["xq"], d["sx_t"], d["wq"], d["sw"], offs)
        ref = O.grouped_mm_fp8(xq, sx, wq, sw, np.cumsum(counts))
        assert_close(to_np(out), ref, TOL_GEMM, "fp8 store")
    elif epi == "swiglu":
        H = 192
        xq, sx, wq, sw, d = _quantised_operands(rng, M, E, 2 * H, 256)
        a, h = ops.grouped_mm_fp8_swiglu(d["xq"], d["sx_t"], d["wq"], d["sw"], offs, None, save_h=True)
        href = O.bf16_round(O.grouped_mm_fp8(xq, sx, wq, sw, np.cumsum(counts)))
        assert_close(to_np(h), href, TOL_GEMM, "fp8 h")
        # the SwiGLU of the kernel's own bf16 h: one bf16 step of h near a
        # row's largest activation already moves that row's a by ~1 %
        assert_close(to_np(a), O.swiglu(to_np(h), None), TOL_GEMM, "fp8 a")
    else:
        aq, sa, wq, sw, d = _quantised_operands(rng, M, E, 256, 384)
        dest = rng.permutation(M).astype(np.int32)
        scale = rng.random(M).astype(np.float32)
        out = ops.grouped_mm_fp8_unpermute(d["xq"], d["sx_t"], d["wq"], d["sw"], offs, f32_dev(scale),
                                           torch.from_numpy(dest).to(DEV), M)
        y = O.grouped_mm_fp8(aq, sa, wq, sw, np.cumsum(counts)) * scale[:, None]
        ref = np.zeros_like(y)
        ref[dest] = y
        assert_close(to_np(out), ref, TOL_GEMM, "fp8 scatter")


@pytest.mark.parametrize("K,score_before,limit", [(1, False, None), (2, False, None), (4, True, 0.05)])
def test_moe_forward_fp8_vs_oracle(pkg, ops, K, score_before, limit):
    import importlib

    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(23 + K)
    T, D, H, E = 512, 512, 256, 8
    x = rand_bf16(rng, (T, D))
    w13 = rand_bf16(rng, (E, 2 * H, D), 0.02)
    w2 = rand_bf16(rng, (E, D, H), 0.02)
    scores, idx = O.router_topk(rng.standard_normal((T, E)).astype(np.float32), K, "softmax", True)
    w13q, s13 = ops.quantize_fp8_blocks(bf16_dev(w13))
    w2q, s2 = ops.quantize_fp8_blocks(bf16_dev(w2))
    announce(f"moe_forward_fp8 K={K} before={score_before} limit={limit}")
    out = F.moe_experts_forward_fp8(bf16_dev(x), f32_dev(scores), torch.from_numpy(idx).to(DEV), w13q, s13,
                                    w2q, s2, E, score_before, limit)
    b13, c13 = O.quantize_fp8_blocks(w13)
    b2, c2 = O.quantize_fp8_blocks(w2)
    ref = O.moe_forward_fp8(x, scores, idx, b13, c13, b2, c2, E, score_before, limit)
    from gpu_util import assert_close

    assert_close(to_np(out), ref, TOL_LAYER, "fp8 layer output")


def test_c5_deepseek_fp8_shard_full_size_sampled(pkg, ops):
    """C5: 32 local experts, D=7168, H=2048, 32768 routed rows with Zipf(1.2)
    load; fp8 weights (128 x 128 scales) and per-token-per-128-channel
    activation scales.  >= 256 sampled rows, including the segment and
    256-row tile edges of every non-empty expert, against the dequantising
    oracle, per row and norm-wise."""
    import importlib

    F = importlib.import_module("torchtitan-ascend_amd.functional")
    rng = np.random.default_rng(55)
    T, D, H, E = 32768, 7168, 2048, 32
    labels = labels_from_counts(zipf_counts(T, E, 1.2, 28, rng), rng).reshape(T, 1)
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(T, D, device=DEV, generator=g).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * H, D, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, D, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    scores = torch.rand(T, 1, device=DEV, generator=g)
    idx = torch.from_numpy(labels).to(DEV)
    announce("C5 full size")
    w13q, s13 = ops.quantize_fp8_blocks(w13)
    w2q, s2 = ops.quantize_fp8_blocks(w2)
    out = F.moe_experts_forward_fp8(x, scores, idx, w13q, s13, w2q, s2, E, False)
    torch.cuda.synchronize()
    # 256 random tokens plus those at the first / last row of every
    # non-empty expert's segment and of every 256-row fp8 tile inside it
    from gpu_util import assert_close, edge_rows

    sidx = O.stable_order(labels, E)
    cnt = O.histogram(labels, E)
    edge_tok = sidx[edge_rows(np.cumsum(cnt), (256,))]
    rows = np.unique(np.concatenate([rng.choice(T, 256, replace=False), edge_tok]))
    assert rows.size >= 256
    ix = labels[rows, 0]
    ref = np.zeros((rows.size, D), np.float32)
    # the oracle one expert at a time: that expert's fp8 weights and block
    # scales, dequantised on the host, against its sampled rows
    for e in np.unique(ix).tolist():
        sel = np.nonzero(ix == e)[0]
        announce(f"C5 full size: oracle, expert {e} ({sel.size} sampled rows of {int(cnt[e])})")
        rt_e = torch.from_numpy(rows[sel]).to(DEV)
        b13, c13 = w13q[e:e + 1].cpu().numpy(), s13[e:e + 1].cpu().numpy()
        b2, c2 = w2q[e:e + 1].cpu().numpy(), s2[e:e + 1].cpu().numpy()
        ref[sel] = O.moe_forward_fp8(to_np(x[rt_e]), scores[rt_e].cpu().numpy(), np.zeros((sel.size, 1), np.int64),
                                     b13, c13, b2, c2, 1, False)
    assert set(np.unique(ix).tolist()) == set(np.nonzero(cnt)[0].tolist())  # every non-empty expert is checked
    rt = torch.from_numpy(rows).to(DEV)
    assert_close(to_np(out[rt]), ref, TOL_LAYER, f"C5 layer output ({rows.size} sampled tokens)")
