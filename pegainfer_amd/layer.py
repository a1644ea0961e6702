"""Composite expert-path layers built from the C-ABI ops.

``RoutedExperts.forward`` is the routed-expert sequence of the reference's
Kimi-K2 decode layer (pegainfer-kimi-k2/src/runner/moe_nccl.rs:152-203):
permutation -> zero-fill -> W13 grouped GEMM (top_k, no weight) -> SwiGLU ->
zero-fill -> W2 grouped GEMM (top_k = 1, bf16 routing weight) -> fp32 top-k
row sum.  With ``combine="weighted"`` the routing weight is applied in the
fp32 combine instead (DeepSeek-V2-Lite order, pegainfer-deepseek-v2-lite/
src/runtime/moe.rs:414-539).  Every buffer is allocated in the constructor;
``forward`` only enqueues kernels on the current stream.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops


def _dev_u8(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(device)


def _dev_bf16(a: np.ndarray, device) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).to(device)
    return t.view(torch.bfloat16)


def package_projection(packed: np.ndarray, scales: np.ndarray, device="cuda") -> ops.MarlinInt4Weight:
    """Upload checkpoint tensors ([E, out, in/2] u8, [E, out, in/32] bf16 bits) and
    repack them on the GPU into the device layout."""
    E, out_dim, half_in = packed.shape
    w = ops.marlin_int4_reorder(_dev_u8(packed, device), _dev_bf16(scales, device), E,
                                2 * half_in, out_dim)
    return w


def package_w13(gate, up, device="cuda") -> ops.MarlinInt4Weight:
    """gate/up = (packed, scales) checkpoint pairs -> fused W13 device package."""
    g = package_projection(*gate, device=device)
    u = package_projection(*up, device=device)
    return ops.marlin_int4_fuse_w13(g, u)


class RoutedExperts:
    """One GPU's share of routed experts with preallocated workspaces."""

    def __init__(self, w13: ops.MarlinInt4Weight, w2: ops.MarlinInt4Weight, *, max_tokens: int,
                 topk: int, block_size: int, global_start: int = 0, device="cuda",
                 extra_splits: int = 1):
        self.w13, self.w2 = w13, w2
        self.E = w13.local_experts
        self.H = w13.in_dim
        self.I = w13.out_dim // 2
        assert w2.in_dim == self.I and w2.out_dim == self.H and w2.local_experts == self.E
        self.topk, self.block_size, self.global_start = topk, block_size, global_start
        self.max_tokens = max_tokens
        self.route_ws = ops.KimiMarlinRouteWorkspace(max_tokens, block_size, device=device,
                                                     topk=topk, local_experts=self.E)
        self.gemm_ws = ops.KimiMarlinWna16Workspace(self.route_ws.max_m_blocks,
                                                    max(2 * self.I, self.H), block_size,
                                                    device=device, extra_splits=extra_splits)
        rows = max_tokens * topk
        bf = dict(dtype=torch.bfloat16, device=device)
        self.w13_out = torch.zeros(rows, 2 * self.I, **bf)
        self.act = torch.zeros(rows, self.I, **bf)
        self.route_out = torch.zeros(rows, self.H, **bf)
        self.routing = None

    def forward(self, hidden: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor,
                out_f32: torch.Tensor, combine: str = "sum", w13_timer=None,
                reference_flow: bool = False, companion=None, routing=None,
                join=None) -> torch.Tensor:
        """Routed-expert forward (moe_nccl.rs:152-203 order: align, W13, SwiGLU, W2
        with the top-k weight, top-k combine).  W13 and SwiGLU are one call unless
        reference_flow is set.

        combine "sum": the weight is applied in the W2 epilogue and rows are summed
        (Kimi); "weighted": W2 without weight and an fmaf-chain combine (DSV2).
        reference_flow=True issues the reference's exact call sequence, zero-fills
        included; the default skips both zero-fills (rows of routes owned by other
        GPUs are never read: W2 reads only local rows, and the combine skips
        non-local routes) and fuses SwiGLU into W13.  The two give the same bits
        whenever the fused and the plain W13 add over the same K shares (prefill
        block sizes; decode grids of two or more W13 workgroups per CU with
        K >= 512); a small decode grid splits K differently, and a W13 sum may then
        differ in the last fp32 bit.
        `w13_timer` (optional) exposes start()/stop(mark) and is called around the
        W13 GEMM launch so a caller can time that kernel with stream events.
        `companion` (optional, prefill block sizes only): a (W13, W2) pair of
        independent problems (ExpertFFN.pair_problems, a shared expert) that run in
        the same two launches as this layer's W13 and W2, dispatched first.
        `routing` (optional): the permutation of topk_idx already built in this
        layer's route workspace (route_from_logits); the align launch is then skipped.
        `join` (optional, not with reference_flow): a (shared, out) pair of bf16
        [T, H] tensors; the combine then writes out = bf16(f(bf16(combine)) + f(shared))
        in the same launch (the DSV2 join, ops.moe_combine_join) instead of out_f32."""
        T = hidden.shape[0]
        rows = T * self.topk
        if routing is None:
            routing = ops.moe_align_block_size(self.route_ws, topk_idx, T, T, self.global_start)
        self.routing = routing
        w13_out = self.w13_out[:rows]
        act = self.act[:rows]
        route_out = self.route_out[:rows]
        if reference_flow:
            w13_out.zero_()
        mark = w13_timer.start() if w13_timer is not None else None
        if companion is not None:
            assert not reference_flow and self.block_size > 16
            ops.wna16_prefill_pair(companion[0], ops.wna16_problem(
                routing, hidden, self.w13, top_k=self.topk, size_m=T, act=act))
            if w13_timer is not None:
                w13_timer.stop(mark)
        elif not reference_flow:
            # SwiGLU in the W13 epilogue (gate and up tiles in one workgroup), routed rows
            # only
            ops.wna16_w13_swiglu(self.gemm_ws, routing, hidden, self.w13, act, top_k=self.topk,
                                 size_m=T)
            if w13_timer is not None:
                w13_timer.stop(mark)
        else:
            ops.wna16_gemm(self.gemm_ws, routing, hidden, self.w13, topk_w, w13_out,
                           top_k=self.topk, mul_topk_weights=False, size_m=T)
            if w13_timer is not None:
                w13_timer.stop(mark)
            ops.kimi_marlin_w13_swiglu(w13_out, act, rows, self.I)
        weighted_in_gemm = combine == "sum"
        if reference_flow:
            route_out.zero_()
        if companion is not None:
            ops.wna16_prefill_pair(companion[1], ops.wna16_problem(
                routing, act, self.w2, top_k=1, size_m=rows, output=route_out,
                topk_weight=topk_w, mul_topk_weights=weighted_in_gemm))
        else:
            ops.wna16_gemm(self.gemm_ws, routing, act, self.w2, topk_w, route_out, top_k=1,
                           mul_topk_weights=weighted_in_gemm, size_m=rows)
        if reference_flow:
            if weighted_in_gemm:
                ops.kimi_marlin_sum_topk_rows_f32(route_out, T, out_f32, self.topk, self.H)
            else:
                ops.weighted_topk_sum_f32(route_out, topk_w, T, out_f32, self.topk, self.H)
        elif join is not None:
            shared, out = join
            ops.moe_combine_join(route_out, topk_idx, None if weighted_in_gemm else topk_w,
                                 shared, out, T, self.topk, self.H, self.global_start, self.E)
            return out
        else:
            ops.moe_combine_local_f32(route_out, topk_idx, None if weighted_in_gemm else topk_w,
                                      T, out_f32, self.topk, self.H, self.global_start, self.E)
        return out_f32

    def route_from_logits(self, logits: torch.Tensor, bias: torch.Tensor, topk_w: torch.Tensor,
                          topk_idx: torch.Tensor, T: int, route_scale: float = 1.0):
        """Kimi router select + permutation in one launch (ops.kimi_route_align), for
        decode batches; returns the routing to pass to forward."""
        return ops.kimi_route_align(self.route_ws, logits, bias, topk_w, topk_idx, T,
                                    self.global_start, route_scale)

    def route_softmax_from_logits(self, logits: torch.Tensor, topk_w: torch.Tensor,
                                  topk_idx: torch.Tensor, T: int):
        """DeepSeek-V2-Lite router + permutation in one launch (ops.dsv2_route_align);
        returns the routing to pass to forward."""
        return ops.dsv2_route_align(self.route_ws, logits, topk_w, topk_idx, T, self.global_start)

    def forward_from_logits(self, hidden: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor,
                            topk_w: torch.Tensor, topk_idx: torch.Tensor, out_f32: torch.Tensor,
                            route_scale: float = 1.0, **kw) -> torch.Tensor:
        """The Kimi router's select stage, then forward: in one fused select +
        permutation launch up to ops.ROUTE_ALIGN_MAX_ROUTES routes (same bits as the
        select and permutation launches, which run above that)."""
        T = hidden.shape[0]
        routing = None
        if fused_route(T, self.topk, logits.shape[-1]):
            routing = self.route_from_logits(logits, bias, topk_w[:T], topk_idx[:T], T,
                                             route_scale)
        else:
            ops.kimi_router_select(logits, bias, topk_w[:T], topk_idx[:T], T, topk=self.topk,
                                   route_scale=route_scale)
        return self.forward(hidden, topk_idx[:T], topk_w[:T], out_f32, routing=routing, **kw)


class DenseW4A16:
    """y = x . dequant(W)^T for one W4A16 matrix (a one-expert grouped GEMM with
    static identity routing)."""

    def __init__(self, w: ops.MarlinInt4Weight, *, max_rows: int, device="cuda",
                 extra_splits: int = 8, block_size: int = None):
        assert w.local_experts == 1
        self.w = w
        self.max_rows = max_rows
        if block_size is None:
            block_size = 8 if max_rows <= 8 else (16 if max_rows <= 16 else 64)
        self.block_size = block_size
        self.route_ws = ops.KimiMarlinRouteWorkspace(max_rows, self.block_size, device=device,
                                                     topk=1, local_experts=1)
        self.gemm_ws = ops.KimiMarlinWna16Workspace(self.route_ws.max_m_blocks, w.out_dim,
                                                    self.block_size, device=device,
                                                    extra_splits=extra_splits)
        self.idx = torch.zeros(max_rows, dtype=torch.int32, device=device)
        self.ones = torch.ones(max_rows, dtype=torch.float32, device=device)
        self._routed_rows = None

    def route(self, rows: int):
        self.routing = ops.moe_align_block_size(self.route_ws, self.idx, rows, rows, 0)
        self._routed_rows = rows

    def forward(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        rows = x.shape[0]
        if self._routed_rows != rows:
            self.route(rows)
        ops.wna16_gemm(self.gemm_ws, self.routing, x, self.w, self.ones, y, top_k=1,
                       mul_topk_weights=False, size_m=rows)
        return y


class KimiSharedExpert:
    """The Kimi-K2 shared expert, a bf16 dense MLP (moe_nccl.rs:107-123): gate/up
    GEMM [2I, H] -> SwiGLU (gate first; silu_mul_fused_cuda,
    csrc/shared/fused_proj.cu:11-31) -> down GEMM [H, I], bf16 `projected` out.
    At decode sizes the gate/up GEMM and the SwiGLU run as one launch
    (dense_w13_swiglu, the same bits as the reference's two calls); from
    PREFILL_TOKENS tokens the reference's prefill sequence runs instead
    (moe_nccl.rs:266-275): the gate/up GEMM into [T, 2I] (gemm_graphsafe, which
    takes hipBLASLt at those sizes), the SwiGLU kernel, the down GEMM."""

    PREFILL_TOKENS = 256

    def __init__(self, gate_up: torch.Tensor, down: torch.Tensor, *, max_tokens: int,
                 device="cuda"):
        assert gate_up.dim() == 2 and down.dim() == 2
        self.gate_up, self.down = gate_up.contiguous(), down.contiguous()
        self.I = gate_up.shape[0] // 2
        self.H = gate_up.shape[1]
        assert tuple(down.shape) == (self.H, self.I)
        bf = dict(dtype=torch.bfloat16, device=device)
        self.act = torch.zeros(max_tokens, self.I, **bf)
        self.h13 = (torch.zeros(max_tokens, 2 * self.I, **bf)
                    if max_tokens >= self.PREFILL_TOKENS else None)

    def forward(self, normed: torch.Tensor, projected: torch.Tensor) -> torch.Tensor:
        T = normed.shape[0]
        if T >= self.PREFILL_TOKENS:
            ops.gemm_graphsafe(self.gate_up, normed, self.h13[:T])
            ops.kimi_marlin_w13_swiglu(self.h13[:T], self.act[:T], T, self.I)
        else:
            ops.dense_w13_swiglu(self.gate_up, normed, self.act[:T])
        ops.gemm_graphsafe(self.down, self.act[:T], projected)
        return projected


def fused_route(tokens: int, topk: int, n_experts: int, softmax: bool = False) -> bool:
    """Whether a layer routes with the fused select + permutation launch.  Kimi
    (sigmoid): whenever its routes fit the one-workgroup sort (ops.ROUTE_ALIGN_MAX_ROUTES)
    and the expert count fits the select (at most 1024); graph-timed against the select
    and permutation launches: 7.8 / 8.6 / 10.2 / 10.4 against 8.6 / 9.4 / 10.2 / 10.3 us
    at 1 / 4 / 16 / 64 tokens (equal from 16 tokens on; one launch less to capture).
    DeepSeek-V2-Lite (softmax): up to 512 routes; at 512 tokens (3072 routes) the fused
    launch took 15.3 against 13.5 us, its 128 workgroups' hand-off and one-workgroup sort
    costing more than the second launch."""
    limit = 512 if softmax else ops.ROUTE_ALIGN_MAX_ROUTES
    return tokens * topk <= limit and n_experts <= 1024


class KimiMoeDecodeLayer:
    """One GPU's Kimi-K2 MoE decode layer (moe_nccl.rs:98-239 without the
    collectives): the shared expert on the normed input, the router select, the
    routed experts (fp32 combine of the local routes) and the residual join
    out = bf16(routed * 2.827 + bf16(hidden + projected)) (kimi_experts.cu:25-39)."""

    def __init__(self, routed: RoutedExperts, shared: KimiSharedExpert, *, n_experts: int = 384,
                 device="cuda"):
        self.routed, self.shared = routed, shared
        T, H = routed.max_tokens, routed.H
        self.projected = torch.zeros(T, H, dtype=torch.bfloat16, device=device)
        self.routed_f32 = torch.zeros(T, H, dtype=torch.float32, device=device)
        self.topk_w = torch.zeros(T, routed.topk, dtype=torch.float32, device=device)
        self.topk_idx = torch.zeros(T, routed.topk, dtype=torch.int32, device=device)

    def forward(self, hidden: torch.Tensor, normed: torch.Tensor, logits: torch.Tensor,
                bias: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        T = hidden.shape[0]
        projected, routed_f32 = self.projected[:T], self.routed_f32[:T]
        self.shared.forward(normed, projected)
        self.routed.forward_from_logits(normed, logits, bias, self.topk_w, self.topk_idx,
                                        routed_f32)
        ops.kimi_residual_add_scaled_f32(hidden, projected, routed_f32, ops.KIMI_K2_ROUTER_SCALE,
                                         out)
        return out


class ExpertFFN:
    """One expert: W13 -> SwiGLU -> W2 (no routing weight), bf16 out."""

    def __init__(self, w13: ops.MarlinInt4Weight, w2: ops.MarlinInt4Weight, *, max_rows: int,
                 device="cuda", extra_splits: int = 8, block_size: int = None):
        self.up = DenseW4A16(w13, max_rows=max_rows, device=device, extra_splits=extra_splits,
                             block_size=block_size)
        self.down = DenseW4A16(w2, max_rows=max_rows, device=device, extra_splits=extra_splits,
                               block_size=block_size)
        self.I = w13.out_dim // 2
        bf = dict(dtype=torch.bfloat16, device=device)
        self.h13 = torch.zeros(max_rows, w13.out_dim, **bf)
        self.act = torch.zeros(max_rows, self.I, **bf)

    def forward(self, x: torch.Tensor, y: torch.Tensor, fused: bool = True) -> torch.Tensor:
        """fused=True: W13 and SwiGLU in one call (block sizes 8/16: K split across
        workgroups, partials summed by the SwiGLU kernel; larger: SwiGLU in the tile
        GEMM's epilogue); fused=False: the reference's sequence, W13 GEMM into h13
        then kimi_marlin_w13_swiglu."""
        rows = x.shape[0]
        if fused:
            if self.up._routed_rows != rows:
                self.up.route(rows)
            ops.wna16_w13_swiglu(self.up.gemm_ws, self.up.routing, x, self.up.w,
                                 self.act[:rows], top_k=1, size_m=rows)
        else:
            self.up.forward(x, self.h13[:rows])
            ops.kimi_marlin_w13_swiglu(self.h13[:rows], self.act[:rows], rows, self.I)
        self.down.forward(self.act[:rows], y)
        return y

    def pair_problems(self, x: torch.Tensor, y: torch.Tensor):
        """This expert's W13 (+ SwiGLU) and W2 as problems for ops.wna16_prefill_pair
        (prefill block sizes): the same GEMMs, and bits, as forward(x, y)."""
        rows = x.shape[0]
        for d in (self.up, self.down):
            if d._routed_rows != rows:
                d.route(rows)
        act = self.act[:rows]
        return (ops.wna16_problem(self.up.routing, x, self.up.w, top_k=1, size_m=rows, act=act),
                ops.wna16_problem(self.down.routing, act, self.down.w, top_k=1, size_m=rows,
                                  output=y))


class Dsv2MoeLayer:
    """DeepSeek-V2-Lite-shaped MoE: softmax top-k routed experts (weights applied
    in the fp32 combine, route order = expert id) plus a shared expert, joined
    as the reference rounds it: bf16(f(bf16(routed_f32)) + f(shared))
    (f32_to_bf16 at nccl_backend.rs:544-545, then the bf16 add at
    runtime/moe.rs:656)."""

    def __init__(self, routed: RoutedExperts, shared: ExpertFFN, device="cuda",
                 overlap_shared: bool = True):
        self.routed, self.shared = routed, shared
        T, H = routed.max_tokens, routed.H
        self.topk_w = torch.zeros(T, routed.topk, dtype=torch.float32, device=device)
        self.topk_idx = torch.zeros(T, routed.topk, dtype=torch.int32, device=device)
        self.routed_f32 = torch.zeros(T, H, dtype=torch.float32, device=device)
        self.shared_out = torch.zeros(T, H, dtype=torch.bfloat16, device=device)
        self.overlap_shared = overlap_shared
        # prefill block sizes overlap in shared launches; the decode kernels use a
        # second stream (default priority, like every stream here), made on first use
        self.pair = (overlap_shared and routed.block_size > 16 and shared.up.block_size > 16
                     and shared.down.block_size > 16)
        self.side = None
        self.device = device

    def _route(self, logits: torch.Tensor, T: int):
        """Softmax top-k select and permutation: one fused launch where the routes fit it
        (then the routing goes to forward), else the select launch (forward permutes)."""
        if fused_route(T, self.routed.topk, logits.shape[-1], softmax=True):
            return self.routed.route_softmax_from_logits(logits, self.topk_w[:T],
                                                         self.topk_idx[:T], T)
        ops.dsv2_router_select(logits, self.topk_w[:T], self.topk_idx[:T], T, self.routed.topk)
        return None

    def forward(self, hidden: torch.Tensor, logits: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """The shared expert does not depend on the routed branch, so by default it
        overlaps with it: its few large workgroups (one expert, 512 rows) share the
        GPU with the routed ones instead of running after them.  At prefill block
        sizes each of its two GEMMs goes into the routed GEMM's launch (one stream,
        its workgroups dispatched first); at decode sizes it runs on a second
        stream that joins before the add.  Either way the kernels' bits are those
        of the serial order."""
        T = hidden.shape[0]
        if self.pair:
            companion = self.shared.pair_problems(hidden, self.shared_out[:T])
            routing = self._route(logits, T)
            # the shared expert is done when W2's launch is, so the combine takes the join
            self.routed.forward(hidden, self.topk_idx[:T], self.topk_w[:T], self.routed_f32[:T],
                                combine="weighted", companion=companion, routing=routing,
                                join=(self.shared_out[:T], out))
            return out
        main = torch.cuda.current_stream()
        if self.overlap_shared and self.side is None:
            self.side = torch.cuda.Stream(device=self.device)
        if self.side is not None:
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                self.shared.forward(hidden, self.shared_out[:T])
        routing = self._route(logits, T)
        self.routed.forward(hidden, self.topk_idx[:T], self.topk_w[:T], self.routed_f32[:T],
                            combine="weighted", routing=routing)
        if self.side is not None:
            main.wait_stream(self.side)
        else:
            self.shared.forward(hidden, self.shared_out[:T])
        ops.moe_join_routed_shared(self.routed_f32[:T], self.shared_out[:T], out)
        return out


def capture_graph(step, warmup: int = 2) -> torch.cuda.CUDAGraph:
    """Capture `step()` (a sequence of this library's launches on the current
    stream) into a HIP graph, as a decode loop replays a layer.  The step is
    run `warmup` times on a side stream first, so every lazily cached device
    query happens outside the capture.  The captured launches contain no
    memset nodes: the default RoutedExperts flow writes every output element it
    later reads and clears nothing."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    return graph
