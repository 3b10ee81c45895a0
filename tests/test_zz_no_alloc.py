"""The allocation-free route entry point (ttamd_moe_route_noalloc) against
ttamd_moe_route with a caller workspace, through the C ABI.

The library's per-device histogram array keeps whatever the previous call
left in it, so the calls run back to back with shrinking inputs: the
largest size the array allows, then a C2-sized routing (Qwen3-30B-A3B,
65,536 labels over 128 experts, with scores), then a tiny int32 case with
out-of-range labels.  Every output must equal ttamd_moe_route's bit for bit
(and the oracle's stable order for the small cases)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _noalloc(labels: torch.Tensor, E: int, scores: torch.Tensor | None):
    import importlib

    _lib = importlib.import_module("torchtitan-ascend_amd._lib")
    M = labels.numel()
    out = {
        "counts": torch.empty(E, dtype=torch.int32, device=DEV),
        "offsets": torch.empty(E + 1, dtype=torch.int32, device=DEV),
        "sorted_indices": torch.empty(M, dtype=torch.int32, device=DEV),
        "inverse": torch.empty(M, dtype=torch.int32, device=DEV),
        "sorted_scores": None if scores is None else torch.empty(M, dtype=torch.float32, device=DEV),
    }

    def p(t):
        return None if t is None else ctypes.c_void_p(t.data_ptr())

    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call():
        _lib.call("ttamd_moe_route_noalloc", p(labels), int(labels.dtype == torch.int64), M, E, p(scores),
                  p(out["counts"]), p(out["offsets"]), p(out["sorted_indices"]), p(out["inverse"]),
                  p(out["sorted_scores"]), stream)
        torch.cuda.synchronize()

    # The first call may load the library's kernels (code objects, not
    # buffers); the second, measured one must leave the device's free memory
    # (any hipMalloc, not only torch's caching allocator) and torch's
    # allocator untouched.  Its outputs are the ones checked.
    call()
    before_torch = torch.cuda.memory_allocated()
    before_free = torch.cuda.mem_get_info()[0]
    call()
    assert torch.cuda.mem_get_info()[0] == before_free
    assert torch.cuda.memory_allocated() == before_torch
    return out


def _check_against_workspace_route(ops, labels, E, scores, oracle_check):
    got = _noalloc(labels, E, scores)
    ref = ops.route(labels, E, scores)
    torch.cuda.synchronize()
    for name in ("counts", "offsets", "sorted_indices", "inverse", "sorted_scores"):
        a, b = got[name], getattr(ref, name)
        if b is None:
            assert a is None
            continue
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy(), err_msg=name)
    if oracle_check:
        lab = labels.cpu().numpy()
        np.testing.assert_array_equal(got["sorted_indices"].cpu().numpy(), O.stable_order(lab, E))
        valid = lab[(lab >= 0) & (lab < E)]
        np.testing.assert_array_equal(got["counts"].cpu().numpy(), np.bincount(valid, minlength=E))


def test_route_noalloc_matches_route_on_shrinking_calls(ops):
    rng = np.random.default_rng(77)
    # 1: the largest histogram the array holds: 2^20 labels over 1023 experts
    #    ((1023 + 1) * 1024 chunks = 2^20 ints)
    E1, M1 = 1023, 1 << 20
    lab1 = torch.from_numpy(rng.integers(0, E1, M1)).to(DEV)
    announce(f"route_noalloc M={M1} E={E1} int64 (array limit)")
    _check_against_workspace_route(ops, lab1, E1, None, oracle_check=False)
    # 2: C2 routing, top-8 of 128 experts for 8192 tokens, with scores
    T, K, E2 = 8192, 8, 128
    lab2 = torch.from_numpy(np.argsort(rng.random((T, E2)), axis=1)[:, :K].astype(np.int64)).to(DEV)
    sc2 = torch.rand(T, K, device=DEV)
    announce(f"route_noalloc M={T * K} E={E2} int64 + scores")
    _check_against_workspace_route(ops, lab2, E2, sc2, oracle_check=True)
    # 3: tiny int32 labels, some outside [0, E) (sorted last), one expert empty
    E3 = 5
    lab3 = np.array([4, 0, 7, 2, 2, -1, 0, 4, 4, 2, 0, 5, 1, 0, 2, 4, 0, 2, 2, 4, 0, 0, 1, 4, 2, 2, 0, 4, 9, 2,
                     1, 0, 2, 4, 4, 2, 0], dtype=np.int32)
    announce(f"route_noalloc M={lab3.size} E={E3} int32, out-of-range labels")
    _check_against_workspace_route(ops, torch.from_numpy(lab3).to(DEV), E3, None, oracle_check=True)
