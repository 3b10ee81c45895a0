"""The torch CPU restatement of the reference op sequence (bench.py's
cpu_baseline leg) agrees with the numpy oracle (CPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from oracle import reference_cpu as R


@pytest.mark.parametrize("K,score_func,norm,before,limit", [(2, "softmax", True, False, None),
                                                            (1, "sigmoid", False, True, None),
                                                            (4, "softmax", True, False, 0.05)])
def test_reference_cpu_matches_oracle(K, score_func, norm, before, limit):
    rng = np.random.default_rng(40 + K)
    T, D, H, E = 96, 64, 32, 8
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    wr = O.bf16_round((rng.standard_normal((E, D)) * 0.2).astype(np.float32))
    w13 = O.bf16_round((rng.standard_normal((E, 2 * H, D)) * 0.1).astype(np.float32))
    w2 = O.bf16_round((rng.standard_normal((E, D, H)) * 0.1).astype(np.float32))
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    sc, idx = R.router(bf(x), bf(wr), K, score_func, norm)
    ref_sc, ref_idx = O.router_topk(O.router_logits(x, wr), K, score_func, norm)
    # selection may differ only on near-ties of bf16 logits; compare the layer on the same routing
    assert (idx.numpy() == ref_idx).mean() > 0.95
    out = R.moe_layer(bf(x), sc, idx, bf(w13), bf(w2), E, before, limit)
    ref = O.moe_forward(x, sc.numpy(), idx.numpy(), w13, w2, E, before, limit)
    assert O.max_rel_err(out.float().numpy(), ref) < 2e-2


def test_reference_cpu_shared_expert_and_labels():
    rng = np.random.default_rng(47)
    T, D, H, E = 40, 32, 16, 4
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w13 = O.bf16_round((rng.standard_normal((E, 2 * H, D)) * 0.1).astype(np.float32))
    w2 = O.bf16_round((rng.standard_normal((E, D, H)) * 0.1).astype(np.float32))
    s13 = O.bf16_round((rng.standard_normal((2 * H, D)) * 0.1).astype(np.float32))
    s2 = O.bf16_round((rng.standard_normal((D, H)) * 0.1).astype(np.float32))
    idx = rng.integers(0, E, (T, 1))
    sc = rng.random((T, 1)).astype(np.float32)
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    out = R.moe_step(bf(x), None, bf(w13), bf(w2), E, 1, "sigmoid", False, True, labels=torch.from_numpy(idx),
                     label_scores=torch.from_numpy(sc), shared=(bf(s13), bf(s2)))
    routed = O.moe_forward(x, sc, idx, w13, w2, E, True)
    ref = O.shared_expert_add(routed, x, s13, s2)
    assert O.max_rel_err(out.float().numpy(), ref) < 2e-2
