"""The one-line JSON contract of bench.py that the round-end driver reads.

* CPU: --gpus above 1 exits with status 2 and one JSON line naming the
  one-GPU limit, before torch is imported.
* GPU: a short C1 run prints one JSON line whose fields have the contract's
  names, types and internal consistency (value = tokens / step time, frac =
  achieved / peak, the stage figures within the step)."""
from __future__ import annotations

import json
import math
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(args, timeout):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=timeout, env={**os.environ, "PYTHONUNBUFFERED": "1"})


def test_more_than_one_gpu_is_refused():
    p = _run(["--gpus", "2"], timeout=60)
    assert p.returncode == 2
    line = json.loads(p.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


@pytest.mark.gpu
def test_bench_line_contract_c1():
    print("[gpu-case] bench.py --config c1 --steps 12 --warmup 2 --cpu-seconds 1", flush=True)
    p = _run(["--config", "c1", "--steps", "12", "--warmup", "2", "--cpu-seconds", "1"], timeout=240)
    assert p.returncode == 0, p.stderr[-2000:]
    b = json.loads(p.stdout.strip().splitlines()[-1])
    base = json.loads((ROOT / "BASELINE.json").read_text())
    assert b["metric"] == base["metric"]
    assert b["n_gpus"] == 1 and b["steps"] == 12 and b["warmup"] == 2
    assert b["higher_is_better"] is True and b["scaling"] == "weak" and b["vs_baseline"] is None
    assert b["dtype"] == "bf16" and "synthetic" in b["data"]
    cfg = b["config"]
    assert isinstance(cfg, dict) and "workload" in cfg and "model" not in cfg
    assert b["ms_per_step"] > 0
    assert math.isclose(b["value"], cfg["tokens"] / (b["ms_per_step"] * 1e-3), rel_tol=0.01)
    assert b["unit"] == "tokens/s"
    r = b["roofline"]
    assert r["bound"] in ("hbm", "mfma") and r["unit"] in ("GB/s", "TFLOP/s")
    assert r["achieved"] > 0 and r["peak"] > 0
    assert math.isclose(r["frac"], r["achieved"] / r["peak"], rel_tol=1e-3, abs_tol=1e-4)
    assert r["traffic"] is None or r["traffic"] > 0
    hv = r["hbm_view"]
    assert hv["unit"] == "GB/s" and math.isclose(hv["frac"], hv["achieved"] / hv["peak"], rel_tol=1e-3, abs_tol=1e-4)
    c = b["cpu_baseline"]
    assert c["value"] > 0 and c["cores"] >= 1 and c["kind"] in ("reference", "port") and c["sample"]
    # one stamped launch per timed step: the stages fit inside the step
    assert sum(b["stage_us"].values()) <= b["ms_per_step"] * 1000.0 * 1.05
