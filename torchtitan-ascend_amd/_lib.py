"""ctypes binding of libttamd_moe.so (the C ABI declared in include/ttamd_moe.h).

The library is loaded after `torch`, so it binds to the HIP runtime torch
already has in the process.  There is no fallback: when the library is
missing, or no GPU is visible, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libttamd_moe.so"
ABI_VERSION = 1

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ttamd_moe.h one to one.
SIGNATURES: dict[str, tuple] = {
    "ttamd_abi_version": (_i32, []),
    "ttamd_last_error": (ctypes.c_char_p, []),
    "ttamd_router_topk": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32, _f32, _f32, _c_void_p, _c_void_p, _c_void_p],
    ),
    "ttamd_router_workspace_bytes": (_sz, [_i64, _i32, _i64]),
    "ttamd_router_fused": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i32, _i32, _i32, _f32, _f32, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_router_backward_workspace_bytes": (_sz, [_i64, _i32, _i64]),
    "ttamd_router_backward": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i32, _i32, _i32, _f32, _f32,
         _c_void_p, _c_void_p, _i32, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_router_route_workspace_bytes": (_sz, [_i64, _i32, _i64, _i32]),
    "ttamd_router_route": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i32, _i32, _i32, _f32, _f32, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p, _sz,
         _c_void_p],
    ),
    "ttamd_route_workspace_bytes": (_sz, [_i64, _i32]),
    "ttamd_moe_route": (
        _i32,
        [_c_void_p, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_moe_route_noalloc": (
        _i32,
        [_c_void_p, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p],
    ),
    "ttamd_moe_gather_rows": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p]
    ),
    "ttamd_moe_dispatch_rows": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "ttamd_moe_token_permute": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i64, _i64, _i32, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _sz, _c_void_p],
    ),
    "ttamd_unpermute_workspace_bytes": (_sz, [_i64, _i32]),
    "ttamd_moe_token_unpermute": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p, _sz, _c_void_p]
    ),
    "ttamd_moe_combine": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "ttamd_moe_token_unpermute_grad": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p, _c_void_p]
    ),
    "ttamd_moe_rowdot": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i64, _i64, _i64, _c_void_p, _c_void_p]
    ),
    "ttamd_moe_group_labels": (_i32, [_c_void_p, _i32, _i32, _i64, _c_void_p, _c_void_p]),
    "ttamd_gemm_workspace_bytes": (_sz, [_i64, _i32]),
    "ttamd_gemm_plan_bytes": (_sz, [_i64, _i32]),
    "ttamd_probe_next_gemm": (_i32, [_c_void_p, _c_void_p]),
    "ttamd_probe_launches": (_i32, [_c_void_p, _i32]),
    "ttamd_grouped_mm": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p, _sz, _c_void_p]
    ),
    "ttamd_grouped_mm_swiglu": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _f32, _c_void_p, _c_void_p, _c_void_p, _sz,
         _c_void_p],
    ),
    "ttamd_grouped_mm_swiglu_gather": (
        _i32,
        [_c_void_p, _i64, _c_void_p, _i32, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _f32, _c_void_p,
         _c_void_p, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_grouped_mm_unpermute": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p,
         _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_moe_experts_forward_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "ttamd_moe_experts_forward": (
        _i32,
        [_c_void_p, _i64, _i64, _i64, _i32, _i32, _c_void_p, _c_void_p, _c_void_p, _i32, _f32, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _sz, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_moe_sum_topk": (_i32, [_c_void_p, _i64, _i64, _i32, _c_void_p, _c_void_p]),
    "ttamd_shared_expert_add": (
        _i32,
        [_c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _f32, _c_void_p, _c_void_p, _c_void_p, _sz,
         _c_void_p],
    ),
    "ttamd_grouped_mm_dgrad": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p, _sz, _c_void_p]
    ),
    "ttamd_grouped_mm_dgrad_swiglu": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _f32, _c_void_p, _c_void_p,
         _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_grouped_mm_wgrad": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _i32, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_quantize_fp8_rows": (
        _i32, [_c_void_p, _c_void_p, _i32, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p]
    ),
    "ttamd_quantize_fp8_blocks": (_i32, [_c_void_p, _i32, _i64, _i64, _c_void_p, _c_void_p, _c_void_p]),
    "ttamd_grouped_mm_fp8": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p,
         _sz, _c_void_p],
    ),
    "ttamd_grouped_mm_fp8_swiglu": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _f32, _c_void_p,
         _c_void_p, _c_void_p, _sz, _c_void_p],
    ),
    "ttamd_grouped_mm_fp8_unpermute": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i64, _i64, _c_void_p, _c_void_p,
         _i64, _c_void_p, _c_void_p, _sz, _c_void_p],
    ),
}

_lib = None
_lock = threading.Lock()


class TtamdError(RuntimeError):
    """A libttamd_moe call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load libttamd_moe.so once (after torch, so the HIP runtime is shared)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (brings torch's libamdhip64 into the process first)

        if not LIB_PATH.exists():
            raise TtamdError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the MoE path has no CPU fallback)"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.ttamd_abi_version()
        if ver != ABI_VERSION:
            raise TtamdError(f"libttamd_moe ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().ttamd_last_error()
        raise TtamdError(msg.decode() if msg else f"libttamd_moe error {rc}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
