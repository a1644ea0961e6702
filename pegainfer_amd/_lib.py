"""ctypes binding of libpega_moe_hip.so (the C ABI declared in include/pega_moe.h).

The library is built in-tree by ``make -C pegainfer_amd/csrc`` (see
``__graft_entry__.build``).  There is no fallback: if the library is missing
or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpega_moe_hip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_LL = ctypes.c_longlong
_F = ctypes.c_float
_B = ctypes.c_bool



class Wna16Problem(ctypes.Structure):
    """pega_wna16_problem (include/pega_moe.h): one problem of pega_wna16_prefill_pair."""
    _fields_ = [("input", _P), ("output", _P), ("act", _P), ("b_qweight", _P),
                ("b_scales", _P), ("sorted_token_ids", _P), ("expert_ids", _P),
                ("num_tokens_post_padded", _P), ("topk_weights", _P),
                ("sorted_token_ids_len", _I), ("moe_block_size", _I), ("top_k", _I),
                ("mul_topk_weights", _I), ("size_m", _I), ("size_n", _I), ("size_k", _I),
                ("local_experts", _I), ("group_size", _I)]


# name -> argument types (return type is int unless listed in _RESTYPE)
SIGNATURES = {
    "pegainfer_kernels_last_error": [],
    "kimi_moe_marlin_align_block_size_cuda": [_P] * 6 + [_I] * 7 + [_P],
    "pega_kimi_route_align": [_P] * 9 + [_I] * 3 + [_F] + [_I] * 5 + [_P],
    "pega_dsv2_route_align": [_P] * 8 + [_I] * 8 + [_P],
    "pega_exp_exact_f32": [_P, _P, _LL, _P],
    "pega_moe_align_block_size": [_P] * 6 + [_I] * 7 + [_P],
    "kimi_deepep_build_marlin_routing_on_stream": [_P] * 4 + [_I] * 5 + [_P],
    "kimi_marlin_int4_reorder_weight_cuda": [_P, _P, _I, _I, _I, _I, _P],
    "kimi_marlin_int4_reorder_scale_cuda": [_P, _P, _I, _I, _I, _I, _P],
    "kimi_marlin_int4_fuse_w13_cuda": [_P] * 6 + [_I] * 4 + [_P],
    "pega_marlin_int4_reorder_weight": [_P, _P, _I, _I, _I, _I, _P],
    "pega_marlin_int4_reorder_scale": [_P, _P, _I, _I, _I, _I, _P],
    "pega_marlin_int4_fuse_w13": [_P] * 6 + [_I] * 4 + [_P],
    "kimi_marlin_wna16_gemm_cuda": [_P] * 10 + [_I] * 4 + [_B] + [_I] * 6 + [_P],
    "pega_wna16_gemm": [_P, _P, _P, _LL] + [_P] * 3 + [_I] + [_P] * 4 + [_I] * 3 + [_B]
    + [_I] * 6 + [_P],
    "kimi_marlin_w13_swiglu_cuda": [_P, _P, _I, _I, _P],
    "kimi_marlin_w13_swiglu_expanded_cuda": [_P, _P, _P, _I, _I, _I, _P],
    "kimi_marlin_sum_topk_rows_f32_cuda": [_P, _P, _I, _I, _I, _P],
    "pega_weighted_topk_sum_f32": [_P, _P, _P, _I, _I, _I, _P],
    "pega_moe_combine_local_f32": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "pega_wna16_w13_swiglu": [_P, _P, _P, _LL, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "pega_wna16_w13_swiglu_noalloc": [_P] * 7 + [_I] * 9 + [_P],
    "kimi_residual_add_scaled_f32_cuda": [_P, _P, _P, _F, _P, _I, _P],
    "kimi_residual_add_scaled_bf16_cuda": [_P, _P, _P, _F, _P, _I, _P],
    "kimi_add_f32_bf16_to_bf16_cuda": [_P, _P, _P, _I, _P],
    "f32_to_bf16_cuda": [_P, _P, _I, _P],
    "add_cuda": [_P, _P, _P, _I, _P],
    "pega_moe_join_routed_shared_bf16": [_P, _P, _P, _I, _P],
    "pega_moe_combine_join_bf16": [_P] * 5 + [_I] * 5 + [_P],
    "pega_kimi_router_select": [_P, _P, _P, _P, _I, _I, _I, _F, _P],
    "kimi_k2_router_noaux_tc_cuda": [_P] * 6 + [_I] * 5 + [_F, _P],
    "pega_dsv2_router_select": [_P, _P, _P, _I, _I, _I, _P],
    "pega_wna16_prefill_pair": [ctypes.POINTER(Wna16Problem), ctypes.POINTER(Wna16Problem), _P],
    "gemm_cuda": [_P, _P, _P, _I, _I, _I, _P],
    "gemm_graphsafe_cuda": [_P, _P, _P, _I, _I, _I, _P],
    "pega_dense_w13_swiglu": [_P, _P, _P, _I, _I, _I, _P],
}
_RESTYPE = {"pegainfer_kernels_last_error": ctypes.c_char_p}

_lib = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, name: str, code: int, reason: str):
        super().__init__(f"{name} failed with status {code}: {reason}")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C pegainfer_amd/csrc` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, _I)
        _lib = L
    return _lib


def last_error() -> str:
    raw = lib().pegainfer_kernels_last_error()
    return raw.decode() if raw else ""


def call(name: str, *args) -> None:
    """Invoke entry point `name`; raise KernelError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise KernelError(name, rc, last_error())
