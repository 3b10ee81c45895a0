"""Write the golden fixtures under tests/golden/ from torch's own CPU routines.

The fixtures pin the CPU oracle (oracle/moe_oracle.py) against computations
that do not share its code: torch.argsort(stable=True), torch.bincount,
torch.topk, torch._grouped_mm (the op the reference calls,
torchtitanturbo/models/common/npu_gmm.py:17-18) and torch autograd.
The reference itself cannot run here (it imports torch_npu and torchtitan,
neither installed), so no fixture comes from it.

Run:  python tests/golden/make_golden.py      (writes *.npz, no pickles)
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent


def _save(name: str, **arrays):
    np.savez_compressed(OUT / f"{name}.npz", **{k: np.asarray(v) for k, v in arrays.items()})


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16)


def routing_cases():
    cases = {}
    g = torch.Generator().manual_seed(0)
    specs = [
        ("uniform", 64, 4, 8),
        ("skewed", 96, 2, 16),
        ("single_expert", 40, 1, 8),
        ("empty_experts", 50, 2, 32),
        ("top8_e128", 32, 8, 128),
        ("one_token", 1, 4, 8),
    ]
    for name, T, K, E in specs:
        if name == "skewed":
            p = torch.tensor([0.5 ** i for i in range(E)])
            lab = torch.multinomial(p / p.sum(), T * K, replacement=True, generator=g).view(T, K)
        elif name == "single_expert":
            lab = torch.full((T, K), 3, dtype=torch.int64)
        elif name == "empty_experts":
            lab = torch.randint(0, 4, (T, K), generator=g) * 5  # only experts 0,5,10,15
        else:
            lab = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
        flat = lab.reshape(-1)
        cases[name] = dict(
            labels=lab.numpy().astype(np.int64),
            num_experts=np.int64(E),
            sorted_indices=torch.argsort(flat, stable=True).numpy().astype(np.int32),
            counts=torch.bincount(flat, minlength=E).numpy().astype(np.int32),
        )
    # labels outside [0, E): this build sorts them after every valid label
    lab = torch.tensor([[2, -1], [7, 0], [2, 9], [1, 2]], dtype=torch.int64)
    E = 8
    flat = lab.reshape(-1)
    bucket = torch.where((flat >= 0) & (flat < E), flat, torch.full_like(flat, E))
    cases["invalid_labels_sort_last"] = dict(
        labels=lab.numpy(), num_experts=np.int64(E),
        sorted_indices=torch.argsort(bucket, stable=True).numpy().astype(np.int32),
        counts=torch.bincount(flat[(flat >= 0) & (flat < E)], minlength=E).numpy().astype(np.int32),
    )
    for name, arr in cases.items():
        _save(f"routing_{name}", **arr)


def permute_cases():
    g = torch.Generator().manual_seed(1)
    T, K, E, D = 24, 2, 6, 16
    tokens = _bf16(torch.randn(T, D, generator=g))
    lab = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    probs = torch.rand(T, K, generator=g)
    flat = lab.reshape(-1)
    sidx = torch.argsort(flat, stable=True)
    permuted = tokens.index_select(0, sidx // K)
    # unpermute: index_copy back to slot order, weight, sum over K (fp32)
    un = torch.zeros(T * K, D)
    un.index_copy_(0, sidx, permuted.float())
    out = (un.view(T, K, D) * probs.unsqueeze(-1)).sum(1)
    out_noprob = un.view(T, K, D).sum(1)
    _save(
        "permute_basic", tokens=tokens.float().numpy(), labels=lab.numpy(), probs=probs.numpy(),
        num_experts=np.int64(E), top_k=np.int64(K), permuted=permuted.float().numpy(),
        sorted_indices=sidx.numpy().astype(np.int32), unpermuted=_bf16(out).float().numpy(),
        unpermuted_noprob=_bf16(out_noprob).float().numpy(),
    )
    # regroup labels of NpuTokenDispatcher._permute (npu_permute.py:68-72)
    ep, E_loc = 3, 4
    counts_group = torch.randint(0, 5, (ep * E_loc,), generator=g)
    counts_group[5] = 0
    labels = torch.arange(E_loc).repeat(ep).repeat_interleave(counts_group)
    _save("regroup_labels", counts_group=counts_group.numpy(), ep=np.int64(ep), num_local_experts=np.int64(E_loc),
          labels=labels.numpy().astype(np.int32))


def router_cases():
    g = torch.Generator().manual_seed(2)
    T, E = 64, 16
    # tie-free logits: distinct values with gaps well above fp32 rounding
    logits = torch.stack([torch.randperm(E, generator=g).float() * 0.37 - 3.0 for _ in range(T)])
    logits = logits + 0.01 * torch.randn(T, E, generator=g)
    bias = torch.randn(E, generator=g) * 0.05
    for func in ("softmax", "sigmoid"):
        s = torch.softmax(logits, dim=-1) if func == "softmax" else torch.sigmoid(logits)
        for K, norm in ((1, False), (4, True), (4, False)):
            v, i = torch.topk(s, K, dim=-1)
            if norm:
                v = v / (v.sum(-1, keepdim=True) + 1e-20)
            _, ib = torch.topk(s + bias, K, dim=-1)
            vb = s.gather(1, ib)
            _save(f"router_{func}_k{K}_{'norm' if norm else 'raw'}", logits=logits.numpy(), top_k=np.int64(K),
                  scores=v.numpy(), indices=i.numpy(), bias=bias.numpy(), scores_bias=vb.numpy(),
                  indices_bias=ib.numpy())


def router_nan_case():
    """Selection values with NaN (a NaN logit, a NaN expert_bias entry):
    torch.topk ranks NaN as the largest value.  Its order among several
    NaNs is implementation-defined, so the expected indices are
    torch.sort(descending=True, stable=True)'s (ties to the lower expert
    id), checked here to pick the same set as torch.topk wherever a row
    holds at most K NaNs (only NaNs where it holds more) and the same order
    wherever it holds at most one."""
    g = torch.Generator().manual_seed(11)
    T, E, K = 32, 16, 4
    logits = torch.stack([torch.randperm(E, generator=g).float() * 0.37 - 3.0 for _ in range(T)])
    logits = logits + 0.01 * torch.randn(T, E, generator=g)
    nan = float("nan")
    for t in range(8):  # one NaN logit
        logits[t, (5 * t + 3) % E] = nan
    for t in range(8, 12):  # two or three
        logits[t, t % E] = nan
        logits[t, (t + 7) % E] = nan
        if t % 2:
            logits[t, (t + 11) % E] = nan
    logits[12] = nan  # the whole row
    bias = torch.randn(E, generator=g) * 0.05
    bias[9] = nan  # expert 9 is always picked first when biased
    s = torch.sigmoid(logits)

    def pick(sel):
        i = torch.sort(sel, dim=-1, descending=True, stable=True).indices[:, :K]
        it = torch.topk(sel, K, dim=-1).indices
        for r in range(T):
            n_nan = int(torch.isnan(sel[r]).sum())
            if n_nan <= K:  # every NaN is picked: the same set
                assert sorted(i[r].tolist()) == sorted(it[r].tolist()), r
            else:  # only NaNs are picked, which ones is torch's choice
                assert bool(torch.isnan(sel[r, it[r]]).all()), r
            if n_nan <= 1:
                assert i[r].tolist() == it[r].tolist(), r
        return i

    i = pick(s)
    ib = pick(s + bias)
    _save("router_sigmoid_k4_nan", logits=logits.numpy(), top_k=np.int64(K), scores=s.gather(1, i).numpy(),
          indices=i.numpy(), bias=bias.numpy(), scores_bias=s.gather(1, ib).numpy(), indices_bias=ib.numpy())


def router_gate_case():
    """F.linear of the router gate (models/qwen3_5/model.py:757), bf16 output."""
    g = torch.Generator().manual_seed(7)
    T, D, E = 48, 128, 40
    x = _bf16(torch.randn(T, D, generator=g))
    w = _bf16(torch.randn(E, D, generator=g) * 0.02)
    logits = _bf16(F.linear(x.float(), w.float()))
    _save("gate_linear", x=x.float().numpy(), w=w.float().numpy(), logits=logits.float().numpy())


def router_backward_cases():
    """Autograd of the upstream router's op sequence on CPU torch
    (models/qwen3_5/model.py:757-765 closed form): bf16 gate Linear, fp32
    softmax / sigmoid, topk, optional renorm (+1e-20), route_scale; d(top)
    random.  Saves the bf16 logits' gradient and dx, dw."""
    g = torch.Generator().manual_seed(11)
    T, D, E = 40, 128, 24
    x0 = _bf16(torch.randn(T, D, generator=g))
    w0 = _bf16(torch.randn(E, D, generator=g) * 0.05)
    for func, K, norm, scale in (("softmax", 4, True, 1.0), ("softmax", 2, False, 2.5), ("sigmoid", 1, False, 1.0),
                                 ("sigmoid", 3, True, 1.5)):
        x = x0.clone().requires_grad_(True)
        w = w0.clone().requires_grad_(True)
        logits = F.linear(x, w)
        logits.retain_grad()
        s = torch.softmax(logits.float(), dim=-1) if func == "softmax" else torch.sigmoid(logits.float())
        top, idx = torch.topk(s, K, dim=-1)
        if norm:
            top = top / (top.sum(dim=-1, keepdim=True) + 1e-20)
        top = top * scale
        gtop = torch.randn(T, K, generator=g)
        top.backward(gtop)
        _save(f"backward_router_{func}_k{K}_{'norm' if norm else 'raw'}", x=x0.float().numpy(), w=w0.float().numpy(),
              logits=logits.detach().float().numpy(), idx=idx.numpy(), grad_top=gtop.numpy(),
              route_scale=np.float32(scale), dlogits=logits.grad.float().numpy(), dx=x.grad.float().numpy(),
              dw=w.grad.float().numpy())


def experts_cases():
    """The reference's op sequence (npu_gmm.py:29-38) on CPU torch, bf16."""
    g = torch.Generator().manual_seed(3)
    E, D, H = 4, 64, 32
    counts = torch.tensor([5, 0, 11, 3], dtype=torch.int64)
    M = int(counts.sum())
    x = _bf16(torch.randn(M, D, generator=g))
    w13 = _bf16(torch.randn(E, 2 * H, D, generator=g) * 0.1)
    w2 = _bf16(torch.randn(E, D, H, generator=g) * 0.1)
    offs = torch.cumsum(counts, 0, dtype=torch.int32)
    for limit in (None, 0.5):
        h = torch._grouped_mm(x, w13.transpose(-2, -1), offs)
        if limit is not None:
            gate, up = h.chunk(2, -1)
            up = torch.clamp(up, min=-limit, max=limit)
            gate = torch.clamp(gate, max=limit)
            h = torch.cat([gate, up], dim=-1)
        gate, up = h.chunk(2, -1)
        a = (F.silu(gate.float()) * up.float()).to(torch.bfloat16)
        y = torch._grouped_mm(a, w2.transpose(-2, -1), offs)
        # fp32 version of the same chain
        h32 = torch.cat([x[s:e].float() @ w13[i].float().T for i, (s, e) in enumerate(zip([0, *offs[:-1].tolist()], offs.tolist()))])
        _save(
            f"experts_{'limit' if limit is not None else 'nolimit'}", x=x.float().numpy(), w13=w13.float().numpy(),
            w2=w2.float().numpy(), counts=counts.numpy(), limit=np.float64(np.nan if limit is None else limit),
            h_bf16=h.float().numpy(), a_bf16=a.float().numpy(), y_bf16=y.float().numpy(), h_f32=h32.numpy(),
        )


def shared_expert_case():
    """The reference block's shared-expert sequence (models/qwen3_5/model.py:794-809)
    on CPU torch in bf16: FeedForward (w1, w3, w2 Linear), sigmoid of the
    Linear(D, 1) gate, then expert_output + shared_expert_output."""
    g = torch.Generator().manual_seed(8)
    T, D, H = 24, 64, 32
    x = _bf16(torch.randn(T, D, generator=g))
    w1 = _bf16(torch.randn(H, D, generator=g) * 0.1)
    w3 = _bf16(torch.randn(H, D, generator=g) * 0.1)
    w2 = _bf16(torch.randn(D, H, generator=g) * 0.1)
    wg = _bf16(torch.randn(1, D, generator=g) * 0.1)
    routed = _bf16(torch.randn(T, D, generator=g))
    shared = F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w3), w2)
    gate_logits = F.linear(x, wg)
    gated = torch.sigmoid(gate_logits) * shared
    _save("shared_expert_gated", x=x.float().numpy(), w13=torch.cat([w1, w3]).float().numpy(),
          w2=w2.float().numpy(), gate_logits=gate_logits.float().numpy().reshape(T),
          routed=routed.float().numpy(), out=(routed + gated).float().numpy(),
          out_ungated=(routed + shared).float().numpy())


def layer_cases():
    """Whole layer fwd + bwd through torch autograd on an fp32 restatement
    (dispatch gather, per-expert F.linear, combine with index_add_ in the
    form of torchtitanturbo/models/qwen3_5/model.py:703-735)."""
    g = torch.Generator().manual_seed(4)
    for name, (T, K, E, D, H, score_before, limit) in {
        "k2_after": (16, 2, 4, 32, 16, False, None),
        "k1_before": (20, 1, 4, 32, 16, True, None),
        "k2_after_limit": (16, 2, 4, 32, 16, False, 0.3),
    }.items():
        x = torch.randn(T, D, generator=g)
        w13 = torch.randn(E, 2 * H, D, generator=g) * 0.2
        w2 = torch.randn(E, D, H, generator=g) * 0.2
        idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
        scores = torch.rand(T, K, generator=g) + 0.1
        dout = torch.randn(T, D, generator=g)
        xs, w13s, w2s, ss = (t.clone().requires_grad_(True) for t in (x, w13, w2, scores))
        out = torch.zeros(T, D)
        for e in range(E):
            tk, kk = torch.where(idx == e)
            if tk.numel() == 0:
                continue
            xi = xs[tk]
            if score_before:
                xi = xi * ss[tk, kk, None]
            h = F.linear(xi, w13s[e])
            gate, up = h.chunk(2, -1)
            if limit is not None:
                up = torch.clamp(up, min=-limit, max=limit)
                gate = torch.clamp(gate, max=limit)
            yi = F.linear(F.silu(gate) * up, w2s[e])
            if not score_before:
                yi = yi * ss[tk, kk, None]
            out = out.index_add(0, tk, yi)
        out.backward(dout)
        _save(
            f"layer_{name}", x=x.numpy(), w13=w13.numpy(), w2=w2.numpy(), idx=idx.numpy(), scores=scores.numpy(),
            dout=dout.numpy(), num_experts=np.int64(E), score_before=np.int64(score_before),
            limit=np.float64(np.nan if limit is None else limit), out=out.detach().numpy(),
            dx=xs.grad.numpy(), dw13=w13s.grad.numpy(), dw2=w2s.grad.numpy(), dscores=ss.grad.numpy(),
        )


def bf16_cases():
    g = torch.Generator().manual_seed(5)
    v = torch.cat([
        torch.randn(4096, generator=g) * 10.0 ** torch.randint(-6, 6, (4096,), generator=g).float(),
        torch.tensor([0.0, -0.0, 1.0, -1.0, 65504.0, 3.4e38, 1e-40, float("inf"), float("-inf")]),
        # exact ties between two bf16 neighbours
        torch.tensor([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8)]),
    ])
    _save("bf16_round", values=v.numpy(), rounded=v.to(torch.bfloat16).float().numpy())


def _fp8_quant_torch(v: torch.Tensor, dims) -> tuple[torch.Tensor, torch.Tensor]:
    """absmax / 448 block recipe with torch's float8_e4m3fn cast (v already
    reshaped so that `dims` span one block)."""
    amax = v.abs().amax(dim=dims, keepdim=True)
    s = amax / 448.0
    q = torch.where(s > 0, v / torch.where(s > 0, s, torch.ones_like(s)), torch.zeros_like(v))
    return q.to(torch.float8_e4m3fn).view(torch.uint8), s


def fp8_cases():
    # every bf16 bit pattern through torch's float8_e4m3fn cast (inputs rebuilt by the test)
    f = (torch.arange(65536, dtype=torch.int32) << 16).view(torch.float32)
    conv = f.to(torch.float8_e4m3fn).view(torch.uint8)
    ties = torch.tensor([
        # exact mid-points between neighbouring e4m3 values, both parities
        1.0 + 1 / 16, 1.0 + 3 / 16, 448.0 + 16.0, 416.0 + 16.0, 2.0 ** -9 * 0.5, 2.0 ** -9 * 1.5,
        2.0 ** -9 * 7.5, 2.0 ** -6 * (1 + 1 / 16), -(1.0 + 1 / 16), 0.0, -0.0, 463.99, 464.01,
    ], dtype=torch.float32)
    _save("fp8_e4m3_convert", bf16_patterns_e4m3=conv.numpy(), ties=ties.numpy(),
          ties_e4m3=ties.to(torch.float8_e4m3fn).view(torch.uint8).numpy(),
          decode=torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy())
    g = torch.Generator().manual_seed(7)
    R, K = 24, 384
    x = torch.randn(R, K, generator=g) * 10.0 ** torch.randint(-3, 3, (R, 1), generator=g).float()
    x[3, 128:256] = 0.0  # an all-zero block
    x = _bf16(x).float()
    q, s = _fp8_quant_torch(x.view(R, K // 128, 128), (2,))
    _save("fp8_quant_rows", x=x.numpy(), bits=q.view(R, K).numpy(), scale=s.view(R, K // 128).numpy())
    E, N = 2, 256
    w = _bf16(torch.randn(E, N, K, generator=g) * 0.02).float()
    w[1, 128:, :128] *= 1e-3
    qw, sw = _fp8_quant_torch(w.view(E, N // 128, 128, K // 128, 128), (2, 4))
    _save("fp8_quant_blocks", w=w.numpy(), bits=qw.view(E, N, K).numpy(),
          scale=sw.view(E, N // 128, K // 128).numpy())
    # fp8 grouped GEMM and a small fp8 layer, computed with torch ops
    counts = torch.tensor([10, 0, 14], dtype=torch.int64)
    M, E3, N3, K3 = int(counts.sum()), 3, 256, 256
    xa = _bf16(torch.randn(M, K3, generator=g)).float()
    wa = _bf16(torch.randn(E3, N3, K3, generator=g) * 0.02).float()
    xq, xs = _fp8_quant_torch(xa.view(M, K3 // 128, 128), (2,))
    wq, ws = _fp8_quant_torch(wa.view(E3, N3 // 128, 128, K3 // 128, 128), (2, 4))
    xd = (xq.view(torch.float8_e4m3fn).float() * xs).view(M, K3)
    wd = (wq.view(torch.float8_e4m3fn).float() * ws).view(E3, N3, K3)
    out = torch.zeros(M, N3)
    start = 0
    for e, c in enumerate(counts.tolist()):
        out[start:start + c] = (xd[start:start + c].double() @ wd[e].double().T).float()
        start += c
    _save("fp8_grouped_mm", xq=xq.view(M, K3).numpy(), sx=xs.view(M, K3 // 128).numpy(),
          wq=wq.view(E3, N3, K3).numpy(), sw=ws.view(E3, N3 // 128, K3 // 128).numpy(),
          counts=counts.numpy(), out=out.numpy())


if __name__ == "__main__":
    torch.manual_seed(0)
    routing_cases()
    permute_cases()
    router_cases()
    router_nan_case()
    router_gate_case()
    router_backward_cases()
    shared_expert_case()
    experts_cases()
    layer_cases()
    bf16_cases()
    fp8_cases()
    print("torch", torch.__version__, "->", sorted(p.name for p in OUT.glob("*.npz")))
