"""ctypes binding of the C ABI declared in ``include/moe_amd.h``.

The library is loaded lazily from ``moe_amd/_moe_amd.so`` (built in-tree by
``moe_amd.build``).  There is no fallback: if the library is missing or a
call fails, a ``RuntimeError`` carrying the library's own message is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("MOE_AMD_LIB", Path(__file__).resolve().parent / "_moe_amd.so"))

MOE_OK = 0
STATUS_NAMES = {
    -1: "MOE_ERR_ARG",
    -2: "MOE_ERR_DTYPE",
    -3: "MOE_ERR_ALIGN",
    -4: "MOE_ERR_WORKSPACE",
    -5: "MOE_ERR_HIP",
    -6: "MOE_ERR_UNSUPPORTED",
}
DTYPE_F32 = 0
DTYPE_BF16 = 1
NUM_TILE_SIZES = 3

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/moe_amd.h one to one.
SIGNATURES: dict[str, tuple] = {
    "moe_amd_abi_version": (_i, []),
    "moe_amd_last_error": (ctypes.c_char_p, []),
    "moe_amd_router_linear": (_i, [_p, _p, _i64, _i, _i, _p, _i, _p]),
    "moe_amd_router_linear_softmax_topk": (
        _i, [_p, _p, _i64, _i, _i, _p, _i, _i, _p, _p, _p, _p, _p]),
    "moe_amd_router_linear_sigmoid_topk": (
        _i, [_p, _p, _i64, _i, _i, _p, _i, _i, _f, _i, _i, _p, _p, _i, _p, _p, _p, _p]),
    "moe_amd_router_linear_backward_dx": (_i, [_p, _p, _i64, _i, _i, _p, _p]),
    "moe_amd_router_linear_backward_dw_workspace_size": (_sz, [_i64, _i, _i]),
    "moe_amd_router_linear_backward_dw": (_i, [_p, _p, _i64, _i, _i, _p, _sz, _p, _p]),
    "moe_amd_router_linear_backward_f32_workspace_size": (_sz, [_i64, _i, _i]),
    "moe_amd_router_linear_backward_f32": (_i, [_p, _p, _p, _i64, _i, _i, _p, _sz, _p, _p, _p]),
    "moe_amd_router_softmax_topk": (_i, [_p, _i, _p, _i64, _i, _i, _i, _p, _p, _p, _p, _p]),
    "moe_amd_router_softmax_topk_backward": (_i, [_p, _p, _p, _p, _i64, _i, _i, _i, _p, _i, _p]),
    "moe_amd_router_sigmoid_topk": (
        _i, [_p, _p, _i64, _i, _i, _i, _f, _i, _i, _p, _p, _i, _p, _p, _p]),
    "moe_amd_router_sigmoid_topk_scores": (
        _i, [_p, _p, _i64, _i, _i, _i, _f, _i, _i, _p, _i, _p, _p, _p]),
    "moe_amd_router_sigmoid_topk_backward": (
        _i, [_p, _p, _p, _i, _p, _i64, _i, _i, _i, _f, _p, _p]),
    "moe_amd_permute_workspace_size": (_sz, [_i64, _i]),
    "moe_amd_tile_plan_size": (_sz, [_i64, _i]),
    "moe_amd_permute": (_i, [_p, _i64, _i, _p, _sz, _p, _p, _p, _p, _p, _sz, _p]),
    "moe_amd_permute_noalloc": (_i, [_p, _i64, _i, _p, _p, _p, _p, _p, _sz, _p]),
    "moe_amd_gemm_gate_up_swiglu": (
        _i, [_p, _p, _i, _p, _p, _p, _i64, _i64, _i, _i, _i, _i, _p, _p, _p]),
    "moe_amd_gemm_down": (_i, [_p, _p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_down_backward_dx_dswiglu": (
        _i, [_p, _p, _p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_down_backward_dw": (_i, [_p, _p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_down_backward_dx_fused_parts": (_i, [_i]),
    "moe_amd_gemm_down_backward_dx_fused": (
        _i, [_p, _p, _i, _p, _p, _p, _p, _p, _i, _i64, _i64, _i, _i, _i, _i, _p, _p, _p, _p]),
    "moe_amd_gemm_down_backward_dw_gathered": (
        _i, [_p, _p, _p, _i, _p, _p, _i64, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_gate_up_backward_dx": (_i, [_p, _p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_gate_up_backward_dw": (
        _i, [_p, _p, _p, _i, _p, _p, _i64, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_down_backward_dw_gathered_accumulate": (
        _i, [_p, _p, _p, _i, _p, _p, _i64, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gemm_gate_up_backward_dw_accumulate": (
        _i, [_p, _p, _p, _i, _p, _p, _i64, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_combine": (_i, [_p, _p, _p, _p, _i, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_combine_backward": (
        _i, [_p, _p, _p, _p, _p, _i, _i64, _i, _i, _i, _i, _p, _p, _p]),
    "moe_amd_weight_grad_reduce": (_i, [_p, _i, _p, _p, _i64, _i, _i, _p, _i, _p]),
    "moe_amd_gather_backward": (_i, [_p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_gather_backward_add": (_i, [_p, _p, _p, _p, _i64, _i, _i, _i, _i, _p, _p]),
    "moe_amd_topk_stats_workspace_size": (_sz, [_i64, _i]),
    "moe_amd_topk_stats": (_i, [_p, _i, _p, _i64, _i, _i, _p, _sz, _p, _p, _p, _p]),
    "moe_amd_seq_stats_workspace_size": (_sz, [_i64, _i, _i]),
    "moe_amd_seq_stats": (_i, [_p, _i, _p, _i64, _i, _i, _i, _p, _sz, _p, _p, _p]),
    "moe_amd_seq_aux_backward": (_i, [_p, _i, _p, _i64, _i, _i, _p, _p]),
    "moe_amd_switch_aux_backward": (_i, [_p, _p, _i64, _i, _i, _p, _p]),
    "moe_amd_update_expert_biases": (_i, [_p, _p, _i, _i, _f, _i, ctypes.c_double, _p, _p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads the shared library once and binds every exported prototype."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"moe_amd HIP library not found at {LIB_PATH}; build it with "
                "`python -m moe_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().moe_amd_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Invokes a status-returning entry point; raises RuntimeError on failure."""
    fn = getattr(load(), name)
    rc = fn(*args)
    if rc != MOE_OK:
        raise RuntimeError(f"{name} failed with {STATUS_NAMES.get(rc, rc)}: {last_error()}")
