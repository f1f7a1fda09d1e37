"""ctypes binding of ``libmlops_mi355x.so`` (declared in ``include/mlops_mi355x.h``).

The library is loaded once, lazily. There is no fallback: when the library is
missing or a GPU entry point fails, the error says so and nothing else runs.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libmlops_mi355x.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t

# name -> (restype, argtypes); must match include/mlops_mi355x.h exactly.
SIGNATURES = {
    "mi355x_last_error": (ctypes.c_char_p, []),
    "mi355x_abi_version": (_I, []),
    "mi355x_router_topk": (_I, [_P, _I, _I, _I, _I, _P, _I, _I, _F, _P, _P, _P, _P]),
    "mi355x_router_stats_workspace_size": (_S, [_I, _I]),
    "mi355x_router_stats": (
        _I,
        [_P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _S, _P],
    ),
    "mi355x_router_topk_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P, _P],
    ),
    "mi355x_router_topk_bwd_split": (
        _I,
        [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P],
    ),
    "mi355x_router_weight_grad_workspace_size": (_S, [_I, _I, _I]),
    "mi355x_router_weight_grad": (_I, [_P, _P, _I, _I, _I, _P, _P, _S, _P]),
    "mi355x_permute_plan_workspace_size": (_S, [_I, _I]),
    "mi355x_permute_plan": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _S, _P]),
    "mi355x_permute_plan_noalloc_max_assignments": (_S, [_I]),
    "mi355x_permute_plan_noalloc": (_I, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "mi355x_permute_quantize_fp8": (_I, [_P, _I, _I, _I, _P, _P, _P, _P]),
    "mi355x_quantize_rows_fp8": (_I, [_P, _I, _I, _I64, _I, _P, _P, _P]),
    "mi355x_swiglu_quantize_fp8": (_I, [_P, _I, _I, _F, _P, _P, _P, _P]),
    "mi355x_quantize_weight_blocks": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "mi355x_transpose_fp8": (_I, [_P, _I, _I, _I, _P, _P]),
    "mi355x_wgrad_padded_rows": (_S, [_I, _I]),
    "mi355x_padded_row_blocks": (_I, [_P, _I, _I, _P, _P]),
    "mi355x_quantize_transpose_fp8": (_I, [_P, _I64, _I, _P, _I, _I, _P, _I, _P, _P, _P]),
    "mi355x_unpermute_combine": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "mi355x_unpermute_sum": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "mi355x_routed_swiglu_bwd": (_I, [_P, _P, _P, _P, _I, _I, _F, _P, _P, _P, _P]),
    "mi355x_routed_swiglu_bwd_rows_fp8": (_I, [_P, _P, _P, _P, _I, _I, _F, _P, _P, _P, _P, _P, _P]),
    "mi355x_swiglu_bwd_quantize_workspace_size": (_S, [_I, _I]),
    "mi355x_swiglu_bwd_quantize": (
        _I,
        [_P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _P, _S, _P],
    ),
    "mi355x_swiglu_bwd_bf16": (
        _I,
        [_P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _S, _P],
    ),
    "mi355x_gemm_fp8_block": (
        _I,
        [_P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _P],
    ),
    "mi355x_rank_product": (_I, [_P, _I, _I, _P, _I, _P, _I, _P, _P]),
    "mi355x_rank_product_workspace_size": (_S, [_I, _I, _I]),
    "mi355x_rank_product_split": (_I, [_P, _I, _I, _P, _I, _P, _I, _I, _P, _P, _S, _P]),
    "mi355x_rank_grad_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "mi355x_rank_grad": (_I, [_P, _I, _I, _P, _I, _P, _I, _I, _I, _P, _P, _S, _P]),
    "mi355x_rank_grad_gather": (_I, [_P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I, _P, _P, _F, _I,
                                     _P, _P, _S, _P]),
    "mi355x_gemm_fp8_block_lora": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _I,
                                        _P, _P]),
    "mi355x_gemm_fp8_block_swiglu": (
        _I,
        [_P, _P, _I, _P, _P, _I, _I, _I, _P, _P, _F, _P, _P, _P, _P],
    ),
    "mi355x_gemm_fp8_block_wgrad": (
        _I,
        [_P, _P, _I, _P, _P, _I, _I, _P, _I, _P, _I, _P],
    ),
    "mi355x_gemm_fp8_block_kmajor": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _P, _P, _P]),
    "mi355x_quantize_token_rows_fp8": (_I, [_P, _I, _I, _P, _P, _P]),
    "mi355x_gemm_fp8_block_gathered": (_I, [_P, _P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _P, _I, _P, _P]),
    "mi355x_gemm_fp8_block_kmajor_gathered": (_I, [_P, _P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _P, _P, _P]),
    "mi355x_gemm_fp8_rowwise_gathered": (_I, [_P, _P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _P, _P, _P]),
    "mi355x_gemm_fp8_rowwise": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _P, _P, _P]),
    "mi355x_quantize_rows_current_fp8": (_I, [_P, _I, _I, _I64, _P, _I, _P, _P, _P]),
    "mi355x_permute_quantize_current_fp8": (_I, [_P, _I, _I, _I, _P, _P, _P, _P]),
    "mi355x_swiglu_quantize_rows_current_fp8": (_I, [_P, _I, _I, _F, _P, _P, _P, _P]),
    "mi355x_gemm_fp8_rowwise_lora": (_I, [_P, _P, _I, _P, _P, _I, _I, _I, _P, _P, _P, _I, _P,
                                          _P]),
    "mi355x_quantize_weights_current_fp8": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _S,
                                                 _P]),
    "mi355x_quantize_weights_current_workspace_size": (_S, [_I, _I, _I]),
}

_lock = threading.Lock()
_lib = None


class NativeError(RuntimeError):
    """A C-ABI entry point returned an error code."""


def library() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY.exists():
                raise RuntimeError(
                    f"{LIBRARY.name} is not built: run `python -m mlops_amd._build` "
                    "(or __graft_entry__.build()); the MI355X MoE path has no fallback"
                )
            lib = ctypes.CDLL(str(LIBRARY))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point; raise ``NativeError`` on failure."""
    lib = library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.mi355x_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed ({status}): {message}")


def query(name: str, *args) -> int:
    """Call a size-returning entry point."""
    return int(getattr(library(), name)(*args))


__all__ = ["LIBRARY", "NativeError", "SIGNATURES", "call", "library", "query"]
