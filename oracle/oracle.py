"""numpy front end of the CPU oracle (``oracle/moe_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- never by the product package
``pegainfer_amd``.  Every function forwards to the C restatement, whose
comments cite the reference file:line it follows.

bf16 tensors travel as ``numpy.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


def build() -> None:
    """Compile the oracle with its Makefile (gcc only, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "oracle_align_block_size": [_P] * 6 + [_I] * 6,
            "oracle_deepep_build_routing": [_P] * 4 + [_I] * 5,
            "oracle_marlin_reorder_weight": [_P, _P, _I, _I, _I],
            "oracle_marlin_unpack_weight": [_P, _P, _I, _I, _I],
            "oracle_marlin_reorder_scale": [_P, _P, _I, _I, _I, _I],
            "oracle_marlin_fuse_w13": [_P] * 6 + [_I] * 4,
            "oracle_wna16_gemm": [_P] * 8 + [_I] * 9,
            "oracle_wna16_gemm_fast": [_P] * 8 + [_I] * 9,
            "oracle_dense_gemm_f32": [_P, _P, _P, _I, _I, _I],
            "oracle_f32_to_bf16_n": [_P, _P, _I],
            "oracle_add_bf16": [_P, _P, _P, _I],
            "oracle_swiglu": [_P, _P, _I, _I],
            "oracle_dense_gemm": [_P, _P, _P, _I, _I, _I],
            "oracle_sum_topk_rows": [_P, _P, _I, _I, _I],
            "oracle_residual_add_scaled_f32": [_P, _P, _P, _F, _P, _I],
            "oracle_residual_add_scaled_bf16": [_P, _P, _P, _F, _P, _I],
            "oracle_add_f32_bf16": [_P, _P, _P, _I],
            "oracle_kimi_router": [_P, _P, _P, _P, _I, _I, _I, _F],
            "oracle_dsv2_router": [_P, _P, _P, _I, _I, _I],
            "oracle_weighted_topk_sum": [_P, _P, _P, _I, _I, _I],
            "oracle_expf": [_F],
            "oracle_f32_to_bf16": [_F],
            "oracle_bf16_to_f32": [ctypes.c_uint16],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _I
        L.oracle_expf.restype = _F
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_bf16_to_f32.restype = _F
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise ValueError(f"{name} rejected its arguments (rc={rc})")


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (vectorised)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- routing
def padded_capacity(route_elems: int, local_experts: int, block_size: int) -> tuple[int, int]:
    """max_padded = routes + E*(bs-1); max_m_blocks = ceil(max_padded/bs)
    (pegainfer-kernels/src/ops/kimi_k2/experts.rs:1500-1511)."""
    max_padded = route_elems + local_experts * (block_size - 1)
    return max_padded, (max_padded + block_size - 1) // block_size


def align_block_size(topk_idx, global_start: int, local_experts: int, block_size: int,
                     max_padded: int | None = None, max_m_blocks: int | None = None):
    topk_idx = np.ascontiguousarray(topk_idx, dtype=np.int32).reshape(-1)
    route_elems = topk_idx.size
    cap_p, cap_b = padded_capacity(route_elems, local_experts, block_size)
    max_padded = cap_p if max_padded is None else max_padded
    max_m_blocks = cap_b if max_m_blocks is None else max_m_blocks
    sorted_ids = np.empty(max_padded, np.int32)
    expert_ids = np.empty(max_m_blocks, np.int32)
    ntp = np.empty(1, np.int32)
    offsets = np.empty(local_experts + 1, np.uint32)
    cursor = np.empty(local_experts, np.uint32)
    _check(lib().oracle_align_block_size(
        _ptr(topk_idx), _ptr(sorted_ids), _ptr(expert_ids), _ptr(ntp), _ptr(offsets),
        _ptr(cursor), route_elems, global_start, local_experts, block_size, max_padded,
        max_m_blocks), "align")
    return dict(sorted_token_ids=sorted_ids, expert_ids=expert_ids,
                num_tokens_post_padded=ntp, expert_offsets=offsets, expert_cursor=cursor)


def deepep_build_routing(psum, num_local_experts, alignment, block_size, max_padded,
                         max_m_blocks):
    psum = np.ascontiguousarray(psum, dtype=np.int32)
    sorted_ids = np.empty(max_padded, np.int32)
    expert_ids = np.empty(max_m_blocks, np.int32)
    ntp = np.empty(1, np.int32)
    _check(lib().oracle_deepep_build_routing(
        _ptr(psum), _ptr(sorted_ids), _ptr(expert_ids), _ptr(ntp), num_local_experts,
        alignment, block_size, max_padded, max_m_blocks), "deepep_build_routing")
    return dict(sorted_token_ids=sorted_ids, expert_ids=expert_ids, num_tokens_post_padded=ntp)


# ---------------------------------------------------------------- repacks
def marlin_reorder_weight(ckpt_u32, in_dim, out_dim, local_experts):
    ck = np.ascontiguousarray(ckpt_u32, dtype=np.uint32).reshape(-1)
    out = np.empty_like(ck)
    _check(lib().oracle_marlin_reorder_weight(_ptr(ck), _ptr(out), in_dim, out_dim,
                                              local_experts), "reorder_weight")
    return out


def marlin_unpack_weight(marlin_u32, in_dim, out_dim, local_experts):
    mw = np.ascontiguousarray(marlin_u32, dtype=np.uint32).reshape(-1)
    out = np.empty_like(mw)
    _check(lib().oracle_marlin_unpack_weight(_ptr(mw), _ptr(out), in_dim, out_dim,
                                             local_experts), "unpack_weight")
    return out


def marlin_reorder_scale(ckpt_bf16, in_dim, out_dim, local_experts, group_size=32):
    ck = np.ascontiguousarray(ckpt_bf16, dtype=np.uint16).reshape(-1)
    out = np.empty_like(ck)
    _check(lib().oracle_marlin_reorder_scale(_ptr(ck), _ptr(out), in_dim, out_dim,
                                             local_experts, group_size), "reorder_scale")
    return out


def marlin_fuse_w13(gate_w, up_w, gate_s, up_s, in_dim, inter, local_experts, group_size=32):
    gw = np.ascontiguousarray(gate_w, dtype=np.uint32).reshape(-1)
    uw = np.ascontiguousarray(up_w, dtype=np.uint32).reshape(-1)
    gs = np.ascontiguousarray(gate_s, dtype=np.uint16).reshape(-1)
    us = np.ascontiguousarray(up_s, dtype=np.uint16).reshape(-1)
    ow = np.empty(gw.size * 2, np.uint32)
    os_ = np.empty(gs.size * 2, np.uint16)
    _check(lib().oracle_marlin_fuse_w13(_ptr(gw), _ptr(uw), _ptr(ow), _ptr(gs), _ptr(us),
                                        _ptr(os_), in_dim, inter, local_experts, group_size),
           "fuse_w13")
    return ow, os_


# ---------------------------------------------------------------- GEMM
def wna16_gemm(input_bf16, qweight_ckpt_u8, scales_ckpt_bf16, routing, topk_weights, *,
               moe_block_size, top_k, mul_topk_weights, size_m, size_n, size_k,
               group_size=32, output=None, threads=1, fast=False):
    """C[sorted_id, :] for every valid routed row; other rows of ``output`` are
    left as given (zeros by default, as the reference's caller zero-fills).
    fast=True runs the vectorised CPU-baseline variant (16 lane sums per dot
    product) instead of the k-ascending checker."""
    a = np.ascontiguousarray(input_bf16, dtype=np.uint16)
    qw = np.ascontiguousarray(qweight_ckpt_u8, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_ckpt_bf16, dtype=np.uint16)
    st = np.ascontiguousarray(routing["sorted_token_ids"], dtype=np.int32)
    ei = np.ascontiguousarray(routing["expert_ids"], dtype=np.int32)
    ntp = np.ascontiguousarray(routing["num_tokens_post_padded"], dtype=np.int32)
    tw = np.ascontiguousarray(topk_weights, dtype=np.float32).reshape(-1)
    if output is None:
        output = np.zeros((size_m * top_k, size_n), np.uint16)
    assert output.flags["C_CONTIGUOUS"] and output.dtype == np.uint16
    fn = lib().oracle_wna16_gemm_fast if fast else lib().oracle_wna16_gemm
    _check(fn(
        _ptr(a), _ptr(output), _ptr(qw), _ptr(sc), _ptr(st), _ptr(ei), _ptr(ntp), _ptr(tw),
        ei.size, moe_block_size, top_k, int(bool(mul_topk_weights)), size_m, size_n, size_k,
        group_size, threads), "wna16_gemm")
    return output


# ---------------------------------------------------------------- dense GEMM
def dense_gemm(w_bf16, x_bf16):
    """Y[n][m] = bf16(sum_k W[m][k] X[n][k]) with fp32 accumulation (the shared
    expert's bf16 GEMM, linear.cu:321-344); W [M, K], X [N, K] -> Y [N, M]."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M, K = w.shape
    N = x.shape[0]
    assert x.shape[1] == K
    y = np.empty((N, M), np.uint16)
    _check(lib().oracle_dense_gemm(_ptr(w), _ptr(x), _ptr(y), M, N, K), "dense_gemm")
    return y


def dense_gemm_f32(w_bf16, x_bf16):
    """Y[n][m] = sum_k W[m][k] X[n][k] in fp32, unrounded (the Kimi router's logits
    GEMM, kimi_router.cu:108-142); W [M, K], X [N, K] -> Y [N, M] float32."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    M, K = w.shape
    N = x.shape[0]
    assert x.shape[1] == K
    y = np.empty((N, M), np.float32)
    _check(lib().oracle_dense_gemm_f32(_ptr(w), _ptr(x), _ptr(y), M, N, K), "dense_gemm_f32")
    return y


def kimi_router_noaux_tc(hidden_bf16, gate_bf16, bias, topk=8, route_scale=1.0):
    """kimi_k2_router_noaux_tc_cuda (kimi_router.cu:148-187): fp32 logits of all
    rows, then the select stage.  Returns (logits, topk_idx, topk_weight)."""
    logits = dense_gemm_f32(gate_bf16, hidden_bf16)
    idx, w = kimi_router(logits, bias, topk=topk, route_scale=route_scale)
    return logits, idx, w


# ---------------------------------------------------------------- elementwise
def f32_to_bf16_n(x_f32):
    """f32_to_bf16_cuda (shared/elementwise.cu:235-244) through the C restatement."""
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    _check(lib().oracle_f32_to_bf16_n(_ptr(x), _ptr(out), x.size), "f32_to_bf16")
    return out


def add_bf16(a_bf16, b_bf16):
    """add_cuda (shared/elementwise.cu:9-21): bf16(f(a) + f(b))."""
    a = np.ascontiguousarray(a_bf16, dtype=np.uint16)
    b = np.ascontiguousarray(b_bf16, dtype=np.uint16)
    assert a.shape == b.shape
    out = np.empty(a.shape, np.uint16)
    _check(lib().oracle_add_bf16(_ptr(a), _ptr(b), _ptr(out), a.size), "add_bf16")
    return out


def dsv2_join(routed_f32, shared_bf16):
    """DeepSeek-V2-Lite routed + shared join as the reference runs it: the fp32
    routed sum to bf16 (f32_to_bf16_hidden_into, nccl_backend.rs:544-545), then
    the bf16 add (add_batch_into, runtime/moe.rs:656)."""
    return add_bf16(f32_to_bf16_n(routed_f32), shared_bf16)

def swiglu(w13_bf16, inter):
    w = np.ascontiguousarray(w13_bf16, dtype=np.uint16)
    rows = w.size // (2 * inter)
    out = np.empty((rows, inter), np.uint16)
    _check(lib().oracle_swiglu(_ptr(w), _ptr(out), rows, inter), "swiglu")
    return out


def sum_topk_rows(route_out_bf16, active_tokens, topk, hidden):
    r = np.ascontiguousarray(route_out_bf16, dtype=np.uint16)
    out = np.empty((active_tokens, hidden), np.float32)
    _check(lib().oracle_sum_topk_rows(_ptr(r), _ptr(out), active_tokens, topk, hidden),
           "sum_topk_rows")
    return out


def residual_add_scaled_f32(hidden, projected, routed_f32, scale):
    h = np.ascontiguousarray(hidden, dtype=np.uint16)
    p = np.ascontiguousarray(projected, dtype=np.uint16)
    r = np.ascontiguousarray(routed_f32, dtype=np.float32)
    out = np.empty_like(h)
    _check(lib().oracle_residual_add_scaled_f32(_ptr(h), _ptr(p), _ptr(r), scale, _ptr(out),
                                                h.size), "residual_f32")
    return out


def residual_add_scaled_bf16(hidden, projected, routed_bf16, scale):
    h = np.ascontiguousarray(hidden, dtype=np.uint16)
    p = np.ascontiguousarray(projected, dtype=np.uint16)
    r = np.ascontiguousarray(routed_bf16, dtype=np.uint16)
    out = np.empty_like(h)
    _check(lib().oracle_residual_add_scaled_bf16(_ptr(h), _ptr(p), _ptr(r), scale,
                                                 _ptr(out), h.size), "residual_bf16")
    return out


def add_f32_bf16(a_f32, b_bf16):
    a = np.ascontiguousarray(a_f32, dtype=np.float32)
    b = np.ascontiguousarray(b_bf16, dtype=np.uint16)
    out = np.empty(b.shape, np.uint16)
    _check(lib().oracle_add_f32_bf16(_ptr(a), _ptr(b), _ptr(out), b.size), "add_f32_bf16")
    return out


# ---------------------------------------------------------------- routers
def kimi_router(logits, bias, topk=8, route_scale=1.0):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    tokens, n_experts = l.shape
    b = np.ascontiguousarray(bias, dtype=np.float32)
    w = np.empty((tokens, topk), np.float32)
    idx = np.empty((tokens, topk), np.int32)
    _check(lib().oracle_kimi_router(_ptr(l), _ptr(b), _ptr(w), _ptr(idx), tokens, n_experts,
                                    topk, route_scale), "kimi_router")
    return idx, w


def dsv2_router(logits, topk=6):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    tokens, n_experts = l.shape
    w = np.empty((tokens, topk), np.float32)
    idx = np.empty((tokens, topk), np.int32)
    _check(lib().oracle_dsv2_router(_ptr(l), _ptr(w), _ptr(idx), tokens, n_experts, topk),
           "dsv2_router")
    return idx, w


def weighted_topk_sum(route_out_bf16, topk_weight, tokens, topk, hidden):
    r = np.ascontiguousarray(route_out_bf16, dtype=np.uint16)
    w = np.ascontiguousarray(topk_weight, dtype=np.float32)
    out = np.empty((tokens, hidden), np.float32)
    _check(lib().oracle_weighted_topk_sum(_ptr(r), _ptr(w), _ptr(out), tokens, topk, hidden),
           "weighted_topk_sum")
    return out


def expf(x: float) -> float:
    return lib().oracle_expf(x)


# ---------------------------------------------------------------- composites
def kimi_moe_layer(hidden_bf16, qw13_ckpt, s13_ckpt, qw2_ckpt, s2_ckpt, topk_idx, topk_w, *,
                   global_start, local_experts, block_size, hidden, inter, topk=8,
                   group_size=32, threads=1, fast=False):
    """The routed-expert sequence of pegainfer-kimi-k2/src/runner/moe_nccl.rs:152-203:
    align -> W13 (top_k=topk, no weight mul) -> SwiGLU -> W2 (top_k=1, weight mul)
    -> fp32 top-k row sum.  W13 checkpoint weights are the fused [E, 2I, H/2]
    (gate rows first).  Returns (routed_f32 [T,H], intermediates dict)."""
    tokens = hidden_bf16.shape[0]
    route_elems = tokens * topk
    routing = align_block_size(topk_idx, global_start, local_experts, block_size)
    w13 = wna16_gemm(hidden_bf16, qw13_ckpt, s13_ckpt, routing, topk_w,
                     moe_block_size=block_size, top_k=topk, mul_topk_weights=False,
                     size_m=tokens, size_n=2 * inter, size_k=hidden, group_size=group_size,
                     threads=threads, fast=fast)
    act = swiglu(w13, inter)
    out = wna16_gemm(act, qw2_ckpt, s2_ckpt, routing, topk_w, moe_block_size=block_size,
                     top_k=1, mul_topk_weights=True, size_m=route_elems, size_n=hidden,
                     size_k=inter, group_size=group_size, threads=threads, fast=fast)
    routed = sum_topk_rows(out, tokens, topk, hidden)
    return routed, dict(routing=routing, w13=w13, act=act, route_out=out)
