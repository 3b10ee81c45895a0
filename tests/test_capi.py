"""The C-ABI library loads and exports what include/ttamd_moe.h declares (CPU).

Only calls that the host-side validation rejects are made here: they return
TTAMD_EINVAL before anything touches a GPU.
"""
from __future__ import annotations

import ctypes
import importlib
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "ttamd_moe.h"
_lib = importlib.import_module("torchtitan-ascend_amd._lib")


def header_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ttamd_\w+)\s*\(", text)))


def test_header_declares_functions():
    names = header_functions()
    assert "ttamd_moe_route" in names and "ttamd_grouped_mm_swiglu" in names
    assert len(names) >= 20


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_binding_covers_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_abi_version():
    assert _lib.load().ttamd_abi_version() == _lib.ABI_VERSION


def _err(rc):
    assert rc == 1, rc
    return _lib.load().ttamd_last_error().decode()


def test_route_rejects_bad_arguments():
    lib = _lib.load()
    ws = ctypes.c_void_p(16)
    # too many experts
    msg = _err(lib.ttamd_moe_route(ctypes.c_void_p(16), 1, 8, 5000, None, None, None, ctypes.c_void_p(16), None,
                                   None, ws, 1 << 20, None))
    assert "num_experts" in msg
    # missing workspace
    msg = _err(lib.ttamd_moe_route(ctypes.c_void_p(16), 1, 8, 4, None, None, None, ctypes.c_void_p(16), None,
                                   None, None, 0, None))
    assert "workspace" in msg
    # scores without sorted_scores
    msg = _err(lib.ttamd_moe_route(ctypes.c_void_p(16), 1, 8, 4, ctypes.c_void_p(16), None, None,
                                   ctypes.c_void_p(16), None, None, ws, 1 << 20, None))
    assert "sorted_scores" in msg


def test_gemm_rejects_bad_shapes():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    ws = lib.ttamd_gemm_workspace_bytes(1024, 8)
    assert ws >= 16 * (1024 // 128 + 8)
    msg = _err(lib.ttamd_grouped_mm(p, p, p, 1024, 8, 100, 64, p, p, ws, None))
    assert "multiple of 128" in msg
    msg = _err(lib.ttamd_grouped_mm_swiglu(p, p, p, 1024, 8, 96, 256, float("nan"), p, None, p, ws, None))
    assert "hidden" in msg
    msg = _err(lib.ttamd_grouped_mm_swiglu(p, p, p, 1024, 8, 128, 256, -1.0, p, None, p, ws, None))
    assert "swiglu_limit" in msg
    msg = _err(lib.ttamd_grouped_mm(ctypes.c_void_p(258), p, p, 1024, 8, 128, 64, p, p, ws, None))
    assert "aligned" in msg
    msg = _err(lib.ttamd_grouped_mm(p, p, None, 1024, 8, 128, 64, p, p, ws, None))
    assert "offs" in msg
    msg = _err(lib.ttamd_grouped_mm(p, p, p, 1024, 8, 128, 64, p, p, 8, None))
    assert "workspace" in msg


def test_rows_reject_bad_hidden():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    msg = _err(lib.ttamd_moe_gather_rows(p, p, None, 10, 10, 12, 1, p, None))
    assert "hidden" in msg
    msg = _err(lib.ttamd_moe_combine(p, p, None, 10, 64, 0, p, None))
    assert "topk" in msg
    msg = _err(lib.ttamd_moe_group_labels(p, 6, 4, 10, p, None))
    assert "multiple" in msg


def test_router_topk_rejects_bad_k():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    msg = _err(lib.ttamd_router_topk(p, None, 4, 8, 9, 0, 0, 0.0, 1.0, p, p, None))
    assert "topk" in msg


@pytest.mark.parametrize("fn", ["ttamd_route_workspace_bytes", "ttamd_gemm_workspace_bytes", "ttamd_gemm_plan_bytes"])
def test_workspace_queries_reject_negative(fn):
    assert getattr(_lib.load(), fn)(-1, 4) == 0


def test_probes_reject_bad_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    msg = _err(lib.ttamd_probe_next_gemm(p, None))
    assert "both events or neither" in msg
    # disarming touches no GPU state
    assert lib.ttamd_probe_next_gemm(None, None) == 0
    msg = _err(lib.ttamd_probe_launches(None, 3))
    assert "events is null" in msg
    msg = _err(lib.ttamd_probe_launches(p, 17))
    assert "num_launches" in msg
    evs = (ctypes.c_void_p * 4)(256, 256, None, 256)
    msg = _err(lib.ttamd_probe_launches(evs, 2))
    assert "events[2] and events[3]" in msg
    assert lib.ttamd_probe_launches(None, 0) == 0


@pytest.mark.parametrize("null_counts, null_offsets", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("want", ["plan", "tokens_per_expert"])
def test_router_route_needs_counts_offsets_for_plan(null_counts, null_offsets, want):
    """A tile plan or the tokens_per_expert accumulator is built from the
    counts / offsets buffers: the call is refused on the host when either
    is missing (nothing reaches the device)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    T, E, D, K = 64, 8, 128, 2
    wsb = lib.ttamd_router_route_workspace_bytes(T, E, D, K)
    planb = lib.ttamd_gemm_plan_bytes(T * K, E)
    counts = None if null_counts else p
    offsets = None if null_offsets else p
    plan = p if want == "plan" else None
    tpe = p if want == "tokens_per_expert" else None
    msg = _err(lib.ttamd_router_route(p, p, None, T, E, D, K, 0, 1, 0.0, 1.0, p, p, counts, offsets, p, None,
                                      None, tpe, plan, planb, p, wsb, None))
    assert "counts and offsets" in msg


def test_route_noalloc_rejects_oversize_and_bad_arguments():
    """The allocation-free route refuses, on the host, sizes whose histogram
    would not fit the library's per-device array, and the usual bad arguments."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # 2^22 labels over 1024 experts: (1025 * 4096) ints > 2^20
    msg = _err(lib.ttamd_moe_route_noalloc(p, 1, 1 << 22, 1024, None, p, p, p, p, None, None))
    assert "workspace" in msg and "ttamd_moe_route" in msg
    msg = _err(lib.ttamd_moe_route_noalloc(p, 1, 8, 5000, None, None, None, p, None, None, None))
    assert "num_experts" in msg
    msg = _err(lib.ttamd_moe_route_noalloc(p, 1, 8, 4, p, None, None, p, None, None, None))
    assert "sorted_scores" in msg
    msg = _err(lib.ttamd_moe_route_noalloc(None, 1, 8, 4, None, None, None, p, None, None, None))
    assert "null" in msg
