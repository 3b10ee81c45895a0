"""Benchmark of the MI355X MoE expert path (BASELINE.json metric).

Default workload (Qwen3-30B-A3B shape, MoE layer
forward, bf16): T=8192 tokens, D=2048, H=768, E=128 experts, top-8 softmax
router with renormalised weights.  One step = router (gate GEMM split over D
+ fp32 softmax + top-k + renorm + histogram) -> stable sort + tile table ->
grouped GEMM w13 + SwiGLU with the permute gather in its loads -> grouped
GEMM w2 + score + un-permute -> K-way sum, on inputs already resident in HBM:
two C-ABI calls (ttamd_router_route, ttamd_moe_experts_forward), six kernel
launches.  In every timed step each kernel takes an event pair as its own
start and end stamps (ttamd_probe_launches, stamped through the kernel's
dispatch), so the stage figures, the GEMM TFLOP/s and `roofline` come from
the timed steps and the stages add up to at most the step.

Prints ONE JSON line (bench contract) with `roofline` for the dominant
kernel (the w13 grouped GEMM) and `cpu_baseline` (the reference op sequence
restated in torch, timed on this host's CPU cores on a bounded sample of the
workload).

Other configs (--config c1|c3|c4|c5) are for development runs; C4 and C5
also time the expert-parallel regroup (`regroup`: the dispatcher's _permute
with each local expert's rows arriving from 8 ranks).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE-layer tokens/s + grouped-GEMM TFLOP/s (% MFMA peak), Qwen3-30B-A3B shape"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0  # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0
EP_REGROUP = 8  # C4/C5: DeepSeek-V3's 256 experts over 8 ranks, 32 local

CONFIGS = {
    "c1": dict(name="C1 Llama4-debugmodel MoE FFN forward", T=2048, D=256, H=512, E=8, K=1, router="sigmoid",
               norm=False, score_before=True, backward=False),
    "c2": dict(name="C2 Qwen3-30B-A3B MoE layer forward", T=8192, D=2048, H=768, E=128, K=8, router="softmax",
               norm=True, score_before=False, backward=False),
    "c3": dict(name="C3 Llama4-Scout MoE layer forward+backward (16 routed experts + 1 shared expert)", T=8192,
               D=5120, H=8192, E=16, K=1, router="sigmoid", norm=False, score_before=True, backward=True,
               shared=True),
    "c4": dict(name="C4 DeepSeek-V3 expert shard forward (Zipf 1.2)", T=32768, D=7168, H=2048, E=32, K=1,
               router="zipf", norm=False, score_before=False, backward=False),
    "c5": dict(name="C5 DeepSeek-V3 expert shard forward, fp8 e4m3 experts (128x128 weight scales, "
                    "1x128 activation scales, Zipf 1.2)", T=32768, D=7168, H=2048, E=32, K=1,
               router="zipf", norm=False, score_before=False, backward=False, fp8=True),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="capture the inference step once as a HIP graph and time its replays (one launch per "
                         "step instead of the host's per-call cost); the roofline probe then runs in extra eager "
                         "steps after the timed ones")
    ap.add_argument("--staged", action="store_true",
                    help="time the op-at-a-time path (router, route, then each GEMM and the sum as its own call) "
                         "instead of the two fused C-ABI calls")
    ap.add_argument("--probe", default="chain", choices=["chain", "none"],
                    help="fused inference configs: chain = every kernel of every timed step stamps its own start "
                         "and end (stage figures from the timed steps); none = bare timed steps, stage figures "
                         "from extra untimed steps")
    ap.add_argument("--param-dtype", default="bf16", choices=["bf16", "fp32"],
                    help="training configs (c3): dtype of the expert weight Parameters; fp32 is the reference's "
                         "(npu_gmm.py:63-64, cast to bf16 per call at :31 / :38), cast once per step here")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device copy (reference for the PMC byte counters) and exit")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="about how much CPU time the reference-CPU baseline's timed runs take")
    ap.add_argument("--settle-ms", type=float, default=400.0,
                    help="untimed steps run for this long before the warm-up steps, so that the GPU's clocks "
                         "have reached their steady state under this load")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs the MoE expert path on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch

    if args.calibrate_copy:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "launches": 3}), flush=True)
        return

    ops = importlib.import_module("torchtitan-ascend_amd.ops")
    F = importlib.import_module("torchtitan-ascend_amd.functional")
    cfg = CONFIGS[args.config]
    T, D, H, E, K = cfg["T"], cfg["D"], cfg["H"], cfg["E"], cfg["K"]
    M = T * K
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    log(f"config {args.config}: T={T} D={D} H={H} E={E} K={K}")

    x = torch.randn(T, D, device=dev).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * H, D, device=dev) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, D, H, device=dev) * 0.02).to(torch.bfloat16)
    w_router = (torch.randn(E, D, device=dev) * 0.02).to(torch.bfloat16)
    zipf_idx = None
    if cfg["router"] == "zipf":
        rng = np.random.default_rng(0)
        r = np.arange(1, 29, dtype=np.float64)
        w = r ** -1.2
        c = np.floor(M * w / w.sum()).astype(np.int64)
        c[0] += M - c.sum()
        counts = np.zeros(E, np.int64)
        counts[rng.permutation(E)[:28]] = c
        lab = rng.permutation(np.repeat(np.arange(E), counts))
        zipf_idx = torch.from_numpy(lab.reshape(T, K)).to(dev)
        zipf_scores = torch.rand(T, K, device=dev)
        # the expert-parallel receive side of the same shard: each local
        # expert's rows arrive split over EP_REGROUP ranks (rank-major)
        counts_group = np.stack([rng.multinomial(int(n), np.full(EP_REGROUP, 1.0 / EP_REGROUP))
                                 for n in counts], axis=1).reshape(-1)

    def router():
        if zipf_idx is not None:
            return zipf_scores, zipf_idx
        # gate nn.Linear (bf16) + fp32 score + top-k + renorm, one kernel
        return ops.router_fused(x, w_router, K, cfg["router"], cfg["norm"])

    def timed_router(ev):
        if ev is None:
            return router()
        pair = ev.setdefault("router", (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)))
        pair[0].record()
        out = router()
        pair[1].record()
        return out

    fp8 = cfg.get("fp8", False)
    if fp8:
        # weights are quantised once, as a checkpoint would be; not timed
        w13q, s13 = ops.quantize_fp8_blocks(w13)
        w2q, s2 = ops.quantize_fp8_blocks(w2)

    shared = cfg.get("shared", False)
    if shared:
        # the always-on shared expert: the same SwiGLU FFN on every token
        sw13 = (torch.randn(2 * H, D, device=dev) * 0.02).to(torch.bfloat16)
        sw2 = (torch.randn(D, H, device=dev) * 0.02).to(torch.bfloat16)

    def step_forward(ev=None):
        if ev is None and not fp8 and not args.staged:
            # The timed step: two C-ABI calls.  ttamd_router_route (gate GEMM
            # + score + top-k + histogram, then the stable order and the
            # GEMMs' tile table) and ttamd_moe_experts_forward (w13 + SwiGLU
            # with the permute gather in its loads, w2 + score + un-permute,
            # K-way sum, both GEMMs on that tile table).
            if zipf_idx is not None:
                r = ops.route(zipf_idx, E, zipf_scores)
            else:
                _, _, r = ops.router_route(x, w_router, K, cfg["router"], cfg["norm"], with_inverse=False)
            out = ops.experts_forward(x, r, w13, w2, K, cfg["score_before"])
            return F.shared_expert_combine(out, x, sw13, sw2) if shared else out
        # stage breakdown: the same kernels one op at a time, events around each
        scores, idx = timed_router(ev)
        if fp8:
            return F.moe_experts_forward_fp8(x, scores, idx, w13q, s13, w2q, s2, E, cfg["score_before"],
                                             stage_events=ev)
        out = F.moe_experts_forward(x, scores, idx, w13, w2, E, cfg["score_before"],
                                    stage_events=ev if ev is not None else {})
        if shared:
            # no autograd here: one fused pass, the shared w2 GEMM adds into out
            pair = ev.setdefault("shared_expert", (torch.cuda.Event(enable_timing=True),
                                                   torch.cuda.Event(enable_timing=True))) if ev is not None else None
            if pair:
                pair[0].record()
            out = F.shared_expert_combine(out, x, sw13, sw2)
            if pair:
                pair[1].record()
        return out

    if args.param_dtype != "bf16" and not cfg["backward"]:
        print(json.dumps({"error": "--param-dtype applies to the training configs (c3)"}))
        sys.exit(2)
    if cfg["backward"]:
        # expert weights as Parameters of --param-dtype (fp32: the reference's
        # master weights, whose bf16 values are the ones the GEMMs use)
        pdt = torch.float32 if args.param_dtype == "fp32" else torch.bfloat16
        w13p = w13.to(pdt).requires_grad_(True)
        w2p = w2.to(pdt).requires_grad_(True)
        dout = torch.randn(T, D, device=dev).to(torch.bfloat16)
        xg = x.clone().requires_grad_(True)
        w_router_p = w_router.clone().requires_grad_(True)
        if shared:
            sw13 = sw13.to(pdt).requires_grad_(True)
            sw2 = sw2.to(pdt).requires_grad_(True)

        def step(ev=None):
            # a training step starts from cleared gradients (zero_grad(set_to_none=True));
            # the router is differentiated with the layer (dx and the gate weight's gradient)
            w13p.grad = w2p.grad = xg.grad = w_router_p.grad = None
            if zipf_idx is not None:
                scores, idx = zipf_scores.clone().requires_grad_(True), zipf_idx
            else:
                scores, idx = F.router(xg, w_router_p, K, cfg["router"], cfg["norm"])
            out = F.moe_experts_forward(xg, scores, idx, w13p, w2p, E, cfg["score_before"])
            if shared:
                sw13.grad = sw2.grad = None
                out = F.shared_expert_combine(out, xg, sw13, sw2)
            out.backward(dout)
            return out
    else:
        def step(ev=None):
            with torch.no_grad():
                return step_forward(ev)

    # Clock settling (untimed, before the W warm-up steps): the GPU raises
    # its clocks only after a few hundred ms of sustained load, so a run
    # with few warm-up steps would otherwise time the ramp (C2: ~0.82 ms per
    # step after 5 steps against ~0.77 at steady clocks).  Steps are queued
    # in batches until --settle-ms of wall time has passed.
    settle_steps = 0
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(10):
            step()
        settle_steps += 10
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"clock settling: {settle_steps} steps; warmup: {args.warmup} steps")
    # Timed region: K steps between two synchronisations, nothing else on the
    # stream but the library's kernel-timing events (recorded on the
    # kernels' stream, below).
    graph = None
    if args.graph:
        if cfg["backward"] or fp8 or args.staged:
            print(json.dumps({"error": "--graph covers the bf16 inference step (two C-ABI calls) only"}))
            sys.exit(2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(max(args.warmup, 3)):
            graph.replay()
        torch.cuda.synchronize()
        log("captured the step as one HIP graph")
    # The fused bf16 inference step (c1, c2, c4) is timed with the
    # launch-chain probe (--probe chain): in timed step i one kernel of the
    # step, kernel i mod n of its n launches (router gate, top-k, rank, w13,
    # w2, K-way sum), takes an event pair as its own start and end stamps
    # through its dispatch; the others run unstamped.  Every stage figure
    # below is then the average over the timed steps that stamped it, and a
    # step carries the cost of one stamped dispatch (a few microseconds;
    # stamping all six costs ~35 us per step).  --probe none times the steps
    # bare and takes the stage figures from extra, untimed fused steps with
    # every kernel stamped.  The other modes (fp8, training, op-at-a-time,
    # graph) time the w13 kernel alone with the GEMM probe.
    fused = graph is None and not (fp8 or args.staged or cfg["backward"])
    probe_mode = args.probe if fused else "gemm"
    permute_first = cfg["score_before"] or D < 128
    router_launches = ["route_hist", "route"] if zipf_idx is not None else ["router_gate", "router_topk", "route"]
    expert_launches = ((["tile_map"] if zipf_idx is not None else []) + (["permute"] if permute_first else [])
                       + ["gemm_w13_swiglu", "gemm_w2_unpermute"] + (["sum_topk"] if K > 1 else []))
    launches = router_launches + expert_launches
    nl = len(launches)

    def new_events(n):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for e in evs:
            e.record()  # creates the HIP events outside the timed region
        return evs

    def one_stamped(pair, j):
        evs = [None] * (2 * nl)
        evs[2 * j], evs[2 * j + 1] = pair
        return evs

    n_probe = args.steps if graph is None else min(args.steps, 50)
    if probe_mode == "chain" and args.steps < 2 * nl:
        print(json.dumps({"error": f"--probe chain needs --steps >= {2 * nl} (each kernel stamped twice)"}))
        sys.exit(2)
    stamps = [tuple(new_events(2)) for _ in range(args.steps)] if probe_mode == "chain" else []
    chains = [one_stamped(stamps[i], i % nl) for i in range(len(stamps))]
    probes = [tuple(new_events(2)) for _ in range(n_probe)] if probe_mode == "gemm" else []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            if probe_mode == "chain":
                ops.probe_launches(chains[i])
            elif probe_mode == "gemm":
                ops.probe_next_gemm(*probes[i])
            step()
    end.record()
    torch.cuda.synchronize()
    if graph is not None:
        # the probe needs the host launch path: extra eager steps, untimed
        for pair in probes:
            ops.probe_next_gemm(*pair)
            step()
        torch.cuda.synchronize()
    ops.probe_next_gemm(None, None)
    ops.probe_launches(None)
    ms = start.elapsed_time(end) / args.steps
    log(f"timed {args.steps} steps: {ms:.3f} ms/step")

    stage_us = {}
    if probe_mode == "chain":
        for j, name in enumerate(launches):
            got = [stamps[i][0].elapsed_time(stamps[i][1]) for i in range(j, args.steps, nl)]
            stage_us[name] = sum(got) * 1000.0 / len(got)
        kernel_us = stage_us["gemm_w13_swiglu"]
        stage_source = (f"launch-chain probe in the {args.steps} timed steps: step i stamps kernel i mod {nl} "
                        f"(its own start / end through its dispatch), each stage averaged over its "
                        f"{args.steps // nl}+ stamped steps")
    elif probe_mode == "none":
        # the same fused steps, untimed, every kernel stamped (queued back to
        # back, one synchronisation at the end)
        full = [new_events(2 * nl) for _ in range(20)]
        torch.cuda.synchronize()
        for c in full:
            ops.probe_launches(c)
            step()
        torch.cuda.synchronize()
        ops.probe_launches(None)
        for j, name in enumerate(launches):
            stage_us[name] = sum(c[2 * j].elapsed_time(c[2 * j + 1]) for c in full) * 1000.0 / len(full)
        kernel_us = stage_us["gemm_w13_swiglu"]
        stage_source = "launch-chain probe in 20 extra, untimed fused steps (timed steps unprobed)"
    else:
        kernel_us = sum(p[0].elapsed_time(p[1]) for p in probes) * 1000.0 / len(probes)
        # Stage breakdown (not part of the timed steps): event pairs around
        # every stage of the op-at-a-time path on the stream the kernels run
        # on, averaged over extra forward passes (no-grad passes for the
        # training configs), queued back to back with one synchronisation at
        # the end, so that no pass starts on an idle GPU.
        n_stage = 20
        with torch.no_grad():  # untimed: the op-at-a-time path's first calls (op registration, workspaces)
            for _ in range(3):
                step_forward({})
        torch.cuda.synchronize()
        passes = []
        for _ in range(n_stage):
            ev = {}
            with torch.no_grad():
                step_forward(ev)
            passes.append(ev)
        torch.cuda.synchronize()
        for ev in passes:
            for name, (s0, s1) in ev.items():
                stage_us[name] = stage_us.get(name, 0.0) + s0.elapsed_time(s1) * 1000.0 / n_stage
        stage_source = f"op-at-a-time path (event pairs around each stage), {n_stage} extra forward passes"
    log(f"stages (us): {json.dumps({k: round(v, 1) for k, v in stage_us.items()})}")

    w13_flops = 4.0 * M * D * H
    w2_flops = 2.0 * M * D * H
    gemm_us = stage_us["gemm_w13_swiglu"] + stage_us["gemm_w2_unpermute"]
    gemm_tflops = (w13_flops + w2_flops) / (gemm_us * 1e-6) / 1e12
    w13_tflops = w13_flops / (stage_us["gemm_w13_swiglu"] * 1e-6) / 1e12
    w2_tflops = w2_flops / (stage_us["gemm_w2_unpermute"] * 1e-6) / 1e12
    if fp8:
        # gather + quantise: read x once, write e4m3 rows and their scales, indices
        permute_bytes = T * D * 2 + M * D + M * (D // 128) * 4 + 8 * M
        permute_us = stage_us["permute_quantize"]
    else:
        # The inference step fuses the gather into the w13 GEMM; the standalone
        # permute kernel (dispatcher API, training path) is timed on its own.
        permute_bytes = T * D * 2 + M * D * 2 + 8 * M
        permute_us = stage_us.get("permute") or time_standalone_permute(ops, router, x, E, K, cfg)
    permute_gbs = permute_bytes / (permute_us * 1e-6) / 1e9
    regroup = None
    if cfg["router"] == "zipf":
        regroup_us = time_regroup(ops, x, counts_group, E)
        regroup_bytes = 2 * M * D * 2 + 8 * M
        regroup_gbs = regroup_bytes / (regroup_us * 1e-6) / 1e9
        regroup = {"ep": EP_REGROUP, "us": round(regroup_us, 2), "bytes": regroup_bytes,
                   "gbs": round(regroup_gbs, 1), "frac_of_hbm": round(regroup_gbs / PEAK_HBM_GBS, 4)}
        log(f"regroup (ep={EP_REGROUP}): {regroup_us:.1f} us, {regroup_gbs:.0f} GB/s")
    peak = PEAK_FP8_TFLOPS if fp8 else PEAK_BF16_TFLOPS

    fwd_flops = 6.0 * M * D * H + (6.0 * T * D * H if cfg.get("shared") else 0.0)
    total_flops = fwd_flops * (3 if cfg["backward"] else 1)
    tokens_per_s = T / (ms * 1e-3)
    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle": {"ms": args.settle_ms, "steps": settle_steps},
        "hip_graph": graph is not None,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 (fp32 block scales, fp32 accumulate)" if fp8 else "bf16",
        "data": "synthetic: x~N(0,1), weights~N(0,0.02), random-init router",
        "config": {"workload": cfg["name"], "tokens": T, "dim": D, "hidden": H, "experts": E, "top_k": K,
                   "router": cfg["router"], "score_before_experts": cfg["score_before"],
                   "backward": cfg["backward"],
                   **({"param_dtype": args.param_dtype} if cfg["backward"] else {})},
        "layer_tflops": round(total_flops / (ms * 1e-3) / 1e12, 1),
        "grouped_gemm_tflops": round(gemm_tflops, 1),
        "grouped_gemm_frac_of_peak": round(gemm_tflops / peak, 4),
        "gemm_w13_tflops": round(w13_tflops, 1),
        "gemm_w2_tflops": round(w2_tflops, 1),
        "permute_us": round(permute_us, 2),
        "permute_gbs": round(permute_gbs, 1),
        "permute_frac_of_hbm": round(permute_gbs / PEAK_HBM_GBS, 4),
        "stage_us": {k: round(v, 2) for k, v in stage_us.items()},
        "stage_source": stage_source,
        "regroup": regroup,
        "roofline": {
            "kernel": roofline_kernel_name(cfg, fp8),
            "bound": "mfma",
            "achieved": round(w13_flops / (kernel_us * 1e-6) / 1e12, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(w13_flops / (kernel_us * 1e-6) / 1e12 / peak, 4),
            "traffic": measured_traffic(args.config),
            "algorithmic_flops_per_launch": w13_flops,
            "avg_launch_us": round(kernel_us, 2),
            # the same launch against the HBM bound (the C2 w13 sits near the
            # MI355X ridge): its algorithmic bytes over its launch time
            "hbm_view": w13_hbm_view(cfg, fp8, T, M, kernel_us, measured_traffic(args.config)),
        },
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, cfg, x, w13, w2, w_router, zipf_idx,
                                              zipf_scores if zipf_idx is not None else None,
                                              (sw13, sw2) if shared else None)
    print(json.dumps(result), flush=True)


def w13_hbm_view(cfg, fp8, T, M, kernel_us, traffic):
    """Algorithmic HBM bytes of one w13 launch and their rate: the token rows
    read once (x [T, D] when the gather is fused into the loads, the routed
    rows [M, D] otherwise; e4m3 plus per-128-channel scales for fp8), the
    weights [E, 2H, D] once (with their 128 x 128 block scales for fp8), the
    activation a [M, H] written (and the pre-activation h [M, 2H] when the
    training step saves it), and 4-byte row ids for the fused gather."""
    D, H, E = cfg["D"], cfg["H"], cfg["E"]
    if fp8:
        nbytes = M * D + M * (D // 128) * 4 + E * 2 * H * D + E * (2 * H // 128) * (D // 128) * 4 + M * H * 2
    else:
        gather = not (cfg["score_before"] or D < 128 or cfg["backward"])
        nbytes = ((T if gather else M) * D * 2 + E * 2 * H * D * 2 + M * H * 2
                  + (M * 2 * H * 2 if cfg["backward"] else 0) + (4 * M if gather else 0))
    gbs = nbytes / (kernel_us * 1e-6) / 1e9
    view = {"algorithmic_bytes": nbytes, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4)}
    if traffic:
        view["measured_traffic_gbs"] = round(traffic / (kernel_us * 1e-6) / 1e9, 1)
    return view


def roofline_kernel_name(cfg, fp8):
    """The w13 kernel the step launches first (the one the probe times)."""
    if fp8:
        return "gg_fp8_kernel<EPI_SWIGLU> (fp8 grouped GEMM w13 + SwiGLU epilogue)"
    if cfg["backward"]:
        return "gg_fwd_kernel<EPI_SWIGLU> (grouped GEMM w13 + SwiGLU epilogue, pre-activation saved)"
    if cfg["score_before"] or cfg["D"] < 128:
        return "gg_fwd_kernel<EPI_SWIGLU> (grouped GEMM w13 + SwiGLU epilogue)"
    return "gg_fwd_kernel<EPI_SWIGLU, GATHER> (permute gather + grouped GEMM w13 + SwiGLU epilogue)"


def time_standalone_permute(ops, router, x, E, K, cfg, reps=20):
    """Average duration (us) of the dispatcher's row permute (ops.permute_rows:
    ttamd_moe_dispatch_rows for top-k > 1, ttamd_moe_gather_rows for top-1) on
    this workload's routing, on the current stream."""
    import torch

    with torch.no_grad():
        scores, idx = router()
        r = ops.route(idx, E, scores.reshape(-1).float())
        scale = scores.reshape(-1).float() if cfg["score_before"] else None
        ops.permute_rows(x, r, K, scale)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s0.record()
        for _ in range(reps):
            ops.permute_rows(x, r, K, scale)
        s1.record()
        torch.cuda.synchronize()
    return s0.elapsed_time(s1) * 1000.0 / reps


def time_regroup(ops, x, counts_group, E, reps=20):
    """Average duration (us) of the dispatcher's expert-parallel regroup
    (HipTokenDispatcher._permute at ep > 1; reference
    NpuTokenDispatcher._permute, npu_permute.py:63-85): the routed rows, received
    rank-major as (rank, local expert) groups, labelled by group_labels and
    moved expert-major by token_permute (stable order + one row gather), on
    the current stream.  Bytes: read and write M rows plus the indices."""
    import numpy as np
    import torch

    cg = torch.from_numpy(counts_group.astype(np.int32)).to(x.device)
    M = x.shape[0]

    def once():
        labels = ops.group_labels(cg, E, M)
        return ops.token_permute(x, labels, E)

    with torch.no_grad():
        for _ in range(3):
            once()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s0.record()
        for _ in range(reps):
            once()
        s1.record()
        torch.cuda.synchronize()
    return s0.elapsed_time(s1) * 1000.0 / reps


def measured_traffic(config):
    """HBM bytes per launch of the w13 kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this workload (null when absent)."""
    path = ROOT / "profiles" / f"gg_fwd_swiglu_{config}_hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(args, cfg, x, w13, w2, w_router, zipf_idx, zipf_scores, shared_w):
    """The reference path's own op sequence (oracle/reference_cpu.py: torch
    router, stable argsort + index_select, torch._grouped_mm bf16 for w13
    and w2, silu(gate) * up, scatter + K-way sum) timed on this host's
    cores: torch.set_num_threads(all cores we may use), one warm-up run, then
    the median of >= 3 runs on a token sample sized to about
    --cpu-seconds of work (the whole workload when that fits)."""
    import subprocess

    import numpy as np
    import torch

    from oracle import reference_cpu as R

    cores = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and 0 < int(share) < cores:
        cores = int(share)  # the CPU share this process is given on the GPU box
    torch.set_num_threads(cores)
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True, timeout=10).stdout
        model = [ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")][0]
    except Exception:  # pragma: no cover
        pass
    T, E, K = cfg["T"], cfg["E"], cfg["K"]
    xc = x.cpu()
    w13c, w2c = w13.cpu(), w2.cpu()
    wrc = w_router.cpu()
    shared_c = None if shared_w is None else (shared_w[0].detach().cpu(), shared_w[1].detach().cpu())
    lab = None if zipf_idx is None else zipf_idx.cpu()
    lsc = None if zipf_scores is None else zipf_scores.cpu()

    def run(n):
        xs = xc[:n]
        if cfg["backward"]:
            xs = xs.clone().requires_grad_(True)
            w13r, w2r = w13c.clone().requires_grad_(True), w2c.clone().requires_grad_(True)
            wrr = wrc.clone().requires_grad_(True)
            sh = None if shared_c is None else tuple(t.clone().requires_grad_(True) for t in shared_c)
        else:
            w13r, w2r, wrr, sh = w13c, w2c, wrc, shared_c
        t0 = time.perf_counter()
        with torch.set_grad_enabled(cfg["backward"]):
            out = R.moe_step(xs, wrr, w13r, w2r, E, K, cfg["router"], cfg["norm"], cfg["score_before"],
                             labels=None if lab is None else lab[:n], label_scores=None if lsc is None else lsc[:n],
                             shared=sh)
            if cfg["backward"]:
                out.backward(torch.ones_like(out))
        return time.perf_counter() - t0

    # size the sample from one small probe run, then warm up once on it
    n0 = min(T, 512)
    dt0 = max(run(n0), 1e-3)
    n = int(min(T, max(n0, n0 * args.cpu_seconds / 3.0 / dt0)))
    n = max(K, n - n % 8)
    log(f"cpu baseline: reference op sequence (torch CPU) on {n} of {T} tokens, {cores} threads, {model}")
    run(n)  # warm-up
    reps = 3 if not cfg["backward"] else 1
    times = sorted(run(n) for _ in range(reps))
    med = float(np.median(times))
    kind = "fwd+bwd" if cfg["backward"] else "forward"
    return {
        "value": round(n / med, 1),
        "unit": "tokens/s" if cfg["router"] != "zipf" else "pairs/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} of the workload's {T} tokens (same inputs and routing), one {kind} of the reference op "
                  f"sequence restated in torch on the CPU (oracle/reference_cpu.py: router F.linear bf16 + fp32 "
                  f"{cfg['router']} + topk, histc + stable argsort + index_select, torch._grouped_mm bf16 w13 / w2, "
                  f"silu(gate)*up, scatter + K-way sum{', shared expert' if shared_c is not None else ''}): "
                  f"1 warm-up, median of {reps} runs = {med:.3f} s (runs {', '.join(f'{t:.3f}' for t in times)}); "
                  f"torch.set_num_threads({cores}); CPU {model}",
    }

if __name__ == "__main__":
    main()
