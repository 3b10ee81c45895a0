"""GPU parity of the routing kernels (router top-k, histogram, stable sort,
permute / unpermute / regroup) against the CPU oracle.  Index outputs are
compared bit-exactly; row moves without arithmetic are bit-exact too."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden_names, load_golden
from gpu_util import DEV, announce, bf16_dev, edge_rows, f32_dev, rand_bf16, to_np, topk_labels, zipf_counts, labels_from_counts
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _check_route(ops, labels_np, E, dtype=torch.int64, scores=None):
    lab = torch.from_numpy(np.ascontiguousarray(labels_np)).to(dtype).to(DEV)
    r = ops.route(lab, E, None if scores is None else f32_dev(scores))
    sidx = O.stable_order(labels_np, E)
    counts = O.histogram(labels_np, E)
    np.testing.assert_array_equal(r.sorted_indices.cpu().numpy(), sidx)
    np.testing.assert_array_equal(r.counts.cpu().numpy(), counts)
    off = O.offsets_from_counts(counts)
    np.testing.assert_array_equal(r.offsets.cpu().numpy()[:E], off[:E])
    np.testing.assert_array_equal(r.inverse.cpu().numpy(), O.inverse_order(sidx))
    if scores is not None:
        np.testing.assert_array_equal(r.sorted_scores.cpu().numpy(), np.asarray(scores, np.float32).reshape(-1)[sidx])
    return r


@pytest.mark.parametrize("name", golden_names("routing_"))
def test_route_golden(ops, name):
    g = load_golden(name)
    announce(f"route golden {name}")
    E = int(g["num_experts"])
    r = _check_route(ops, g["labels"], E)
    np.testing.assert_array_equal(r.sorted_indices.cpu().numpy(), g["sorted_indices"])


@pytest.mark.parametrize(
    "T,K,E,dtype",
    [
        (8192, 8, 128, torch.int64),  # Qwen3-30B-A3B shape
        (8192, 8, 128, torch.int32),
        (2048, 1, 8, torch.int64),  # Llama4 debug (config 1)
        (8192, 1, 16, torch.int64),  # Llama4 Scout (config 3)
        (3, 2, 1024, torch.int64),
        (1000, 6, 64, torch.int32),
    ],
)
def test_route_uniform_bit_exact(ops, T, K, E, dtype):
    rng = np.random.default_rng(T * 31 + K * 7 + E)
    announce(f"route T={T} K={K} E={E} {dtype}")
    lab = topk_labels(T, K, E, rng)
    sc = rng.random((T, K)).astype(np.float32)
    _check_route(ops, lab, E, dtype, sc)


def test_route_zipf_skew_bit_exact(ops):
    """DeepSeek-V3 shard shape (config 4): 32768 pairs, 32 experts, Zipf(1.2), 4 empty."""
    rng = np.random.default_rng(4)
    counts = zipf_counts(32768, 32, 1.2, 28, rng)
    lab = labels_from_counts(counts, rng)
    announce("route zipf 32768x32")
    r = _check_route(ops, lab, 32)
    assert int((r.counts == 0).sum()) == 4


def test_route_edge_cases(ops):
    announce("route edge cases")
    _check_route(ops, np.zeros((0,), np.int64), 8)  # no tokens
    _check_route(ops, np.full((5000,), 3, np.int64), 8)  # one expert takes everything
    rng = np.random.default_rng(9)
    lab = rng.integers(-3, 12, 3000)  # labels outside [0, 8) sort last
    r = _check_route(ops, lab, 8)
    assert int(r.offsets[-1]) == int(((lab >= 0) & (lab < 8)).sum())


def test_route_deterministic(ops):
    rng = np.random.default_rng(10)
    lab = torch.from_numpy(topk_labels(4096, 8, 128, rng)).to(DEV)
    announce("route determinism")
    a = ops.route(lab, 128).sorted_indices
    for _ in range(3):
        assert torch.equal(a, ops.route(lab, 128).sorted_indices)


@pytest.mark.parametrize("T,K,E,D", [(512, 8, 128, 2048), (300, 2, 6, 64), (64, 1, 4, 7168)])
def test_token_permute_unpermute(ops, T, K, E, D):
    rng = np.random.default_rng(T + D)
    tok = rand_bf16(rng, (T, D))
    lab = topk_labels(T, K, E, rng)
    probs = rng.random((T, K)).astype(np.float32)
    announce(f"token_permute T={T} K={K} E={E} D={D}")
    permuted, sidx = ops.token_permute(bf16_dev(tok), torch.from_numpy(lab).to(DEV), E)
    ref_p, ref_s = O.permute(tok, lab, K, E)
    np.testing.assert_array_equal(sidx.cpu().numpy(), ref_s)
    np.testing.assert_array_equal(to_np(permuted), ref_p)
    un = ops.token_unpermute(permuted, sidx, None, K)
    np.testing.assert_array_equal(to_np(un), O.unpermute(ref_p, ref_s, None, K))
    unp = ops.token_unpermute(permuted, sidx, f32_dev(probs), K)
    assert O.max_rel_err(to_np(unp), O.unpermute(ref_p, ref_s, probs, K)) < 1e-2
    gout = rand_bf16(rng, (T, D))
    gp, gprobs = ops.token_unpermute_grad(bf16_dev(gout), sidx, f32_dev(probs), permuted, K, need_probs_grad=True)
    ref_gp, ref_gprobs = O.unpermute_grad(gout, ref_s, probs, K, permuted=ref_p)
    np.testing.assert_array_equal(to_np(gp), ref_gp)
    assert O.max_rel_err(gprobs.cpu().numpy(), ref_gprobs) < 1e-4


def test_unpermute_top1_round_trip(ops):
    """NPUMoeTokenUnpermute contract (npu_permute.py:15-53): unpermute(permute(x)) == x."""
    pkg = __import__("importlib").import_module("torchtitan-ascend_amd")
    rng = np.random.default_rng(5)
    T, D, E = 777, 256, 9
    x = bf16_dev(rand_bf16(rng, (T, D))).requires_grad_(True)
    lab = torch.from_numpy(rng.integers(0, E, T)).to(DEV)
    announce("unpermute round trip")
    permuted, sidx = ops.token_permute(x.detach(), lab, E)
    permuted.requires_grad_(True)
    back = pkg.HIPMoeTokenUnpermute.apply(permuted, sidx, x.shape)
    assert torch.equal(back, x.detach())
    g = torch.randn_like(back)
    back.backward(g)
    np.testing.assert_array_equal(to_np(permuted.grad), to_np(g)[sidx.cpu().numpy()])
    empty = torch.empty(0, D, dtype=torch.bfloat16, device=DEV)
    assert pkg.HIPMoeTokenUnpermute.apply(empty, sidx[:0], empty.shape).numel() == 0


def test_gather_rows_score_before_bit_exact(ops):
    """Dispatch with score_before_experts: bf16(float(x) * score), rounded once."""
    rng = np.random.default_rng(6)
    T, K, E, D = 1024, 2, 16, 512
    x = rand_bf16(rng, (T, D))
    lab = topk_labels(T, K, E, rng)
    sc = rng.random((T, K)).astype(np.float32)
    announce("gather_rows score-before")
    r = ops.route(torch.from_numpy(lab).to(DEV), E, f32_dev(sc))
    routed = ops.gather_rows(bf16_dev(x), r.sorted_indices, K, r.sorted_scores)
    sidx = O.stable_order(lab, E)
    ref = O.bf16_round(x[sidx // K] * sc.reshape(-1)[sidx][:, None])
    np.testing.assert_array_equal(to_np(routed), ref)


@pytest.mark.parametrize("T,K,E,D,before", [(1024, 2, 16, 512, True), (777, 8, 128, 2048, False),
                                             (300, 1, 4, 7168, False), (5, 3, 8, 8, True)])
def test_dispatch_rows_bit_exact(ops, T, K, E, D, before):
    """Scatter-form permute from the inverse map: the same routed rows as the
    gather form and as the oracle (bit-exact), with and without the score."""
    rng = np.random.default_rng(T + K + D)
    x = rand_bf16(rng, (T, D))
    lab = topk_labels(T, K, E, rng)
    sc = rng.random((T, K)).astype(np.float32)
    announce(f"dispatch_rows T={T} K={K} D={D} before={before}")
    r = ops.route(torch.from_numpy(lab).to(DEV), E, f32_dev(sc))
    xs = bf16_dev(x)
    routed = ops.dispatch_rows(xs, r.inverse, K, f32_dev(sc.reshape(-1)) if before else None)
    gathered = ops.gather_rows(xs, r.sorted_indices, K, r.sorted_scores if before else None)
    assert torch.equal(routed, gathered)
    sidx = O.stable_order(lab, E)
    ref = x[sidx // K]
    if before:
        ref = O.bf16_round(ref * sc.reshape(-1)[sidx][:, None])
    np.testing.assert_array_equal(to_np(routed), ref)


def test_regroup_permute_matches_reference_semantics(pkg):
    """NpuTokenDispatcher._permute (npu_permute.py:63-85) with synthetic
    (rank, expert) counts: ep=4 ranks x 8 local experts, one GPU."""
    rng = np.random.default_rng(12)
    ep, E_loc, D = 4, 8, 256
    counts_group = rng.integers(0, 40, ep * E_loc)
    counts_group[[3, 17]] = 0
    M = int(counts_group.sum())
    x = rand_bf16(rng, (M, D))
    disp = pkg.HipTokenDispatcher.Config(num_experts=E_loc * ep, top_k=1).build()
    announce("regroup permute ep=4")
    shape, permuted, pidx, ntpe = disp._permute(bf16_dev(x), torch.from_numpy(counts_group).to(DEV), ep, E_loc)
    ref_p, ref_s, ref_n = O.regroup_permute(x, counts_group, ep, E_loc)
    np.testing.assert_array_equal(pidx.cpu().numpy(), ref_s)
    np.testing.assert_array_equal(to_np(permuted), ref_p)
    np.testing.assert_array_equal(ntpe.cpu().numpy(), ref_n)
    back = disp._unpermute(permuted, shape, pidx)
    np.testing.assert_array_equal(to_np(back), x)


def test_regroup_permute_full_size_c4(pkg):
    """The expert-parallel regroup at C4's full size: M = 32768 rows of
    D = 7168 received from ep = 8 ranks for 32 local experts (Zipf(1.2) loads,
    four experts empty), NpuTokenDispatcher._permute's contract
    (npu_permute.py:63-85).  The permuted indices equal the oracle's stable
    order bit for bit, the rows at every expert-segment edge plus a random
    sample moved bit for bit, and each column's sum of the bf16 bit patterns
    (an integer checksum of all rows, invariant under any permutation) is
    unchanged."""
    rng = np.random.default_rng(21)
    ep, E_loc, M, D = 8, 32, 32768, 7168
    counts = zipf_counts(M, E_loc, 1.2, 28, rng)
    counts_group = np.stack([rng.multinomial(int(n), np.full(ep, 1.0 / ep)) for n in counts], axis=1).reshape(-1)
    gen = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(M, D, device=DEV, generator=gen).to(torch.bfloat16)
    disp = pkg.HipTokenDispatcher.Config(num_experts=E_loc * ep, top_k=1).build()
    announce(f"regroup permute full size M={M} D={D} ep={ep} E_loc={E_loc}")
    _, permuted, pidx, ntpe = disp._permute(x, torch.from_numpy(counts_group).to(DEV), ep, E_loc)
    ref_s = O.stable_order(O.group_labels(counts_group, E_loc, M), E_loc)
    got_s = pidx.cpu().numpy()
    np.testing.assert_array_equal(got_s, ref_s)
    np.testing.assert_array_equal(ntpe.cpu().numpy(), counts)
    rows = np.unique(np.concatenate([edge_rows(np.cumsum(counts)), rng.choice(M, 256, replace=False)]))
    ri = torch.from_numpy(rows).to(DEV)
    src = torch.from_numpy(ref_s[rows].astype(np.int64)).to(DEV)
    assert torch.equal(permuted[ri], x[src])
    colsum = lambda t: t.view(torch.int16).to(torch.int64).sum(0)  # noqa: E731
    assert torch.equal(colsum(permuted), colsum(x))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_regroup_permute_autograd(pkg, dtype):
    """_permute is differentiable (torch_npu.npu_moe_token_permute is): the
    gradient of routed_input is the permuted-row gradient scattered back,
    grad[sorted[j]] = g[j] (oracle: inverse of the regroup order).  Rows move
    bit for bit in the input's dtype, fp32 included; _unpermute's backward is
    the matching gather."""
    rng = np.random.default_rng(13)
    ep, E_loc, D = 2, 6, 128
    counts_group = rng.integers(0, 30, ep * E_loc)
    counts_group[4] = 0
    M = int(counts_group.sum()) + 3  # 3 rows past the grouped ones (label E_loc, sorted last)
    x = (rng.standard_normal((M, D)) * 3).astype(np.float32)
    if dtype == torch.bfloat16:
        x = O.bf16_round(x)
    disp = pkg.HipTokenDispatcher.Config(num_experts=E_loc * ep, top_k=1).build()
    xd = torch.from_numpy(x).to(DEV).to(dtype).requires_grad_(True)
    announce(f"regroup permute autograd {dtype}")
    shape, permuted, pidx, _ = disp._permute(xd, torch.from_numpy(counts_group).to(DEV), ep, E_loc)
    assert permuted.dtype == dtype and permuted.grad_fn is not None
    _, ref_s, _ = O.regroup_permute(x, counts_group, ep, E_loc)
    np.testing.assert_array_equal(pidx.cpu().numpy(), ref_s)
    np.testing.assert_array_equal(permuted.detach().float().cpu().numpy(), x[ref_s])
    g = (rng.standard_normal((M, D))).astype(np.float32)
    permuted.backward(torch.from_numpy(g).to(DEV).to(dtype))
    ref_grad = np.empty_like(g)
    ref_grad[ref_s] = g
    want = torch.from_numpy(ref_grad).to(dtype).float().numpy()
    np.testing.assert_array_equal(xd.grad.float().cpu().numpy(), want)
    # _unpermute(_permute(x)) == x bit for bit, and its backward gathers
    y = permuted.detach().requires_grad_(True)
    back = disp._unpermute(y, shape, pidx)
    assert back.dtype == dtype
    np.testing.assert_array_equal(back.detach().float().cpu().numpy(), xd.detach().float().cpu().numpy())
    back.backward(torch.from_numpy(g).to(DEV).to(dtype))
    np.testing.assert_array_equal(y.grad.float().cpu().numpy(),
                                  torch.from_numpy(g).to(dtype).float().numpy()[ref_s])


def test_group_labels_golden(ops):
    g = load_golden("regroup_labels")
    announce("group labels golden")
    lab = ops.group_labels(torch.from_numpy(g["counts_group"]).to(DEV), int(g["num_local_experts"]), g["labels"].size + 2)
    np.testing.assert_array_equal(lab.cpu().numpy(), O.group_labels(g["counts_group"], int(g["num_local_experts"]), g["labels"].size + 2))
    np.testing.assert_array_equal(lab.cpu().numpy()[:-2], g["labels"])


@pytest.mark.parametrize("name", golden_names("router_"))
def test_router_topk_golden(ops, name):
    g = load_golden(name)
    func = "softmax" if "softmax" in name else "sigmoid"
    norm = name.endswith("norm")
    K = int(g["top_k"])
    announce(f"router golden {name}")
    s, i = ops.router_topk(f32_dev(g["logits"]), K, func, norm)
    np.testing.assert_array_equal(i.cpu().numpy(), g["indices"])
    np.testing.assert_allclose(s.cpu().numpy(), g["scores"], rtol=2e-6, atol=1e-7)
    s, i = ops.router_topk(f32_dev(g["logits"]), K, func, False, expert_bias=f32_dev(g["bias"]))
    np.testing.assert_array_equal(i.cpu().numpy(), g["indices_bias"])
    np.testing.assert_allclose(s.cpu().numpy(), g["scores_bias"], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,E,K,func,norm", [(8192, 128, 8, "softmax", True), (8192, 16, 1, "sigmoid", False),
                                             (1000, 256, 8, "sigmoid", True), (33, 1024, 16, "softmax", False)])
def test_router_topk_vs_oracle(ops, T, E, K, func, norm):
    rng = np.random.default_rng(E + K)
    # distinct logits with gaps >= 0.04, so no two scores are within rounding
    logits = (np.argsort(rng.random((T, E)), axis=1) * 0.05 - E * 0.025).astype(np.float32)
    logits += rng.uniform(-0.005, 0.005, (T, E)).astype(np.float32)
    announce(f"router T={T} E={E} K={K} {func}")
    s, i = ops.router_topk(f32_dev(logits), K, func, norm, route_scale=1.5)
    rs, ri = O.router_topk(logits, K, func, norm, route_scale=1.5)
    np.testing.assert_array_equal(i.cpu().numpy(), ri)
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-5, atol=1e-7)


def test_router_ties(ops):
    logits = np.array([[1.0, 3.0, 3.0, 0.0, 3.0], [2.0, 2.0, 2.0, 2.0, 2.0]], np.float32)
    announce("router ties")
    _, i = ops.router_topk(f32_dev(logits), 3, "sigmoid")
    np.testing.assert_array_equal(i.cpu().numpy(), [[1, 2, 4], [0, 1, 2]])


@pytest.mark.parametrize("T,E,K,func,n_open", [(100, 16, 8, "sigmoid", 4), (77, 128, 8, "softmax", 3),
                                               (40, 256, 16, "sigmoid", 5)])
def test_router_masked_experts(ops, T, E, K, func, n_open):
    """Experts masked by an expert bias of -inf stay pickable after every
    finite one, in expert-id order: the order of a stable sort of the
    selection values, the oracle's rule (torch.topk returns -inf entries
    too).  With K above the number of unmasked experts every pick is still a
    distinct expert, scored with its unbiased router score.  Both top-k
    kernels: over given logits, and the fused router (on its own bf16
    logits; E = 128 and 256 take its full-row path, E = 16 the ragged one)."""
    rng = np.random.default_rng(E + n_open)
    bias = np.full(E, -np.inf, np.float32)
    bias[rng.permutation(E)[:n_open]] = rng.standard_normal(n_open).astype(np.float32) * 0.01
    norm = True
    announce(f"router masked experts T={T} E={E} K={K} {func} open={n_open}")
    logits = rng.standard_normal((T, E)).astype(np.float32)
    s, i = ops.router_topk(f32_dev(logits), K, func, norm, expert_bias=f32_dev(bias))
    rs, ri = O.router_topk(logits, K, func, norm, expert_bias=bias)
    got = i.cpu().numpy()
    np.testing.assert_array_equal(got, ri)
    assert all(len(set(r)) == K for r in got.tolist())
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=2e-6, atol=1e-7)
    D = 256
    x = rand_bf16(rng, (T, D))
    w = rand_bf16(rng, (E, D), 0.05)
    s, i, lg = ops.router_fused(bf16_dev(x), bf16_dev(w), K, func, norm, expert_bias=f32_dev(bias),
                                return_logits=True)
    rs, ri = O.router_topk(to_np(lg), K, func, norm, expert_bias=bias)
    got = i.cpu().numpy()
    np.testing.assert_array_equal(got, ri)
    assert all(len(set(r)) == K for r in got.tolist())
    np.testing.assert_allclose(s.cpu().numpy(), rs, rtol=1e-5, atol=1e-7)


def _bf16_ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 1e-30)))
    return np.exp2(e - 7)


@pytest.mark.parametrize("T,D,E,K,func,norm,bias", [
    (1000, 2048, 128, 8, "softmax", True, False),   # Qwen3-30B-A3B router shape
    (2048, 256, 8, 1, "sigmoid", False, False),     # Llama4-debugmodel
    (300, 512, 16, 1, "sigmoid", False, False),     # Llama4-Scout expert count
    (257, 384, 256, 8, "sigmoid", True, True),      # DeepSeek-V3 count, expert bias
    (33, 128, 60, 4, "softmax", False, False),      # ragged token tile, E not a block multiple
])
def test_router_fused_vs_oracle(ops, T, D, E, K, func, norm, bias):
    """Fused gate GEMM + top-k: the bf16 logits match the oracle's F.linear to
    one bf16 step, and the selection on the kernel's own logits is the
    oracle's, bit for bit (scores to fp32 rounding)."""
    rng = np.random.default_rng(T + E)
    x = rand_bf16(rng, (T, D))
    w = rand_bf16(rng, (E, D), 0.02)
    eb = (rng.standard_normal(E) * 0.05).astype(np.float32) if bias else None
    announce(f"router_fused T={T} D={D} E={E} K={K} {func} norm={norm} bias={bias}")
    s, i, lg = ops.router_fused(bf16_dev(x), bf16_dev(w), K, func, norm, route_scale=1.25,
                                expert_bias=None if eb is None else f32_dev(eb), return_logits=True)
    lg = to_np(lg)
    ref_lg = O.router_logits(x, w)
    d = np.abs(lg - ref_lg)
    # one bf16 step of the result plus the fp32 dot-product error bound
    # gamma_D * sum |x||w| (summation order differs from the oracle's)
    gamma = D * 2.0 ** -24 / (1 - D * 2.0 ** -24)
    bound = _bf16_ulp(ref_lg) * 1.01 + gamma * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(d <= bound)
    assert (d > 0).mean() < 0.02
    rs, ri = O.router_topk(lg, K, func, norm, route_scale=1.25, expert_bias=eb)
    np.testing.assert_array_equal(to_np(i), ri)
    np.testing.assert_allclose(to_np(s), rs, rtol=2e-6, atol=1e-7)
    # without the logits output: same result
    s2, i2 = ops.router_fused(bf16_dev(x), bf16_dev(w), K, func, norm, route_scale=1.25,
                              expert_bias=None if eb is None else f32_dev(eb))
    np.testing.assert_array_equal(to_np(i2), ri)
    np.testing.assert_array_equal(to_np(s2), to_np(s))


def test_router_fused_matches_two_stage(ops):
    """On the Qwen3-30B-A3B shape the fused router picks what the two-stage
    path (gate GEMM, then ttamd_router_topk) picks on the same logits."""
    rng = np.random.default_rng(5)
    T, D, E, K = 8192, 2048, 128, 8
    x = bf16_dev(rand_bf16(rng, (T, D)))
    w = bf16_dev(rand_bf16(rng, (E, D), 0.02))
    announce("router_fused vs two-stage, C2 shape")
    s, i, lg = ops.router_fused(x, w, K, "softmax", True, return_logits=True)
    s2, i2 = ops.router_topk(lg.float(), K, "softmax", True)
    assert torch.equal(i, i2)
    torch.testing.assert_close(s, s2, rtol=2e-6, atol=1e-7)
