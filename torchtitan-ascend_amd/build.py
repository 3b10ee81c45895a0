"""Build libttamd_moe.so (the C-ABI library of the MoE expert path) in-tree.

Compiles every source under csrc/ with hipcc for gfx950 only and links one
shared library next to this file.  Run as a script or through
`build_library()`; `__graft_entry__.build()` calls it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libttamd_moe.so"
OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
DEVICE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the MoE library needs the ROCm toolchain")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile and link libttamd_moe.so; returns its path."""
    hipcc = _hipcc()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [obj_dir / (s.name + ".o") for s in srcs]
    cmds = []
    for src, obj in zip(srcs, objs):
        lang = ["-x", "hip"]
        cmds.append([hipcc, *lang, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 1, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    out = PKG_DIR / LIB_NAME
    tmp = PKG_DIR / (LIB_NAME + ".tmp")
    link = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    _run(link)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build_library(verbose=True)
