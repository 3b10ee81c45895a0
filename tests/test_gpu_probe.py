"""The kernel timing probes the bench's figures come from
(ttamd_probe_launches, ttamd_probe_next_gemm): each stamped launch gets its
own start and end (positive duration), consecutive launches of one stream
are stamped in launch order without overlapping, a NULL pair leaves its
launch unstamped, and the GEMM probe stamps the grouped GEMM's main kernel
(not the router kernels before it).  The stamped work must also give the
same results as unstamped work."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce

pytestmark = pytest.mark.gpu
ops = importlib.import_module("torchtitan-ascend_amd.ops")

T, D, H, E, K = 4096, 2048, 768, 32, 4


def _inputs():
    g = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn(T, D, device=DEV, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, D, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * H, D, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, D, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    return x, wr, w13, w2


def _events(n):
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in evs:
        e.record()
    torch.cuda.synchronize()
    return evs


def _step(x, wr, w13, w2):
    _, _, r = ops.router_route(x, wr, K, "softmax", True, with_inverse=False)
    return ops.experts_forward(x, r, w13, w2, K, False)


def test_launch_chain_stamps_each_kernel_in_order():
    """The fused step is six launches (gate GEMM, top-k, rank, w13, w2, the
    K-way sum); a chain over all six stamps them in launch order."""
    x, wr, w13, w2 = _inputs()
    with torch.no_grad():
        ref = _step(x, wr, w13, w2)
        torch.cuda.synchronize()
        evs = _events(12)
        announce("probe chain over the six kernels of the fused step")
        ops.probe_launches(evs)
        out = _step(x, wr, w13, w2)
        torch.cuda.synchronize()
    ops.probe_launches(None)
    assert torch.equal(out, ref)
    dur = [evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(6)]
    gaps = [evs[2 * i + 1].elapsed_time(evs[2 * i + 2]) for i in range(5)]
    assert all(d > 0 for d in dur), dur
    assert all(g >= -1e-3 for g in gaps), gaps  # the next kernel starts after this one ends
    # the two grouped GEMMs dominate the step
    assert min(dur[3], dur[4]) > max(dur[0], dur[1], dur[2], dur[5]), dur


def test_launch_chain_null_pairs_and_gemm_probe():
    """Only the launch given a pair is stamped (here the w2 GEMM, launch 4);
    the GEMM probe alone stamps the first grouped-GEMM main kernel (w13)."""
    x, wr, w13, w2 = _inputs()
    with torch.no_grad():
        _step(x, wr, w13, w2)
        a, b = _events(2)
        evs = [None] * 12
        evs[8], evs[9] = a, b
        announce("probe chain with one stamped launch")
        ops.probe_launches(evs)
        _step(x, wr, w13, w2)
        torch.cuda.synchronize()
        t_w2 = a.elapsed_time(b)
        c, d = _events(2)
        announce("GEMM probe")
        ops.probe_next_gemm(c, d)
        _step(x, wr, w13, w2)
        torch.cuda.synchronize()
        t_w13 = c.elapsed_time(d)
        # a full chain of the same step for comparison
        full = _events(12)
        ops.probe_launches(full)
        _step(x, wr, w13, w2)
        torch.cuda.synchronize()
    ops.probe_launches(None)
    ops.probe_next_gemm(None, None)
    f_w13 = full[6].elapsed_time(full[7])
    f_w2 = full[8].elapsed_time(full[9])
    assert t_w2 > 0 and t_w13 > 0
    # the same kernels: within a factor that excludes the router kernels
    # (each a few percent of a GEMM here) and a whole step
    assert 0.5 * f_w2 < t_w2 < 2.0 * f_w2, (t_w2, f_w2)
    assert 0.5 * f_w13 < t_w13 < 2.0 * f_w13, (t_w13, f_w13)
    assert np.isfinite([t_w2, t_w13, f_w2, f_w13]).all()


def test_probe_is_per_host_thread():
    """A probe armed in one host thread is not taken by launches from
    another (for example torch's autograd worker): the armed GEMM stamp lands
    on the arming thread's next step, after the other thread's step."""
    import threading

    x, wr, w13, w2 = _inputs()
    with torch.no_grad():
        _step(x, wr, w13, w2)
        torch.cuda.synchronize()
        a, b = _events(2)
        announce("GEMM probe armed in the main thread, a step from another thread")
        ops.probe_next_gemm(a, b)

        def other():
            with torch.no_grad():
                _step(x, wr, w13, w2)
            torch.cuda.synchronize()

        t = threading.Thread(target=other)
        t.start()
        t.join()
        mid = torch.cuda.Event(enable_timing=True)
        mid.record()
        _step(x, wr, w13, w2)  # the main thread's next GEMM takes the probe
        torch.cuda.synchronize()
    ops.probe_next_gemm(None, None)
    assert mid.elapsed_time(a) > 0, "the probe stamped the other thread's launch"
    assert a.elapsed_time(b) > 0
