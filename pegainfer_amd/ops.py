"""Host-side mirror of the reference's Kimi-K2 expert ops over the C ABI.

Reference: pegainfer-kernels/src/ops/kimi_k2/experts.rs (Rust wrappers around
the CUDA entry points).  Names, argument meaning, shape guards and error
behaviour follow that file; tensors are torch device tensors (bf16 travels as
torch.bfloat16 or as its uint16 bit pattern), and every op enqueues on
torch's current HIP stream without synchronising or allocating, except the
workspace constructors (which allocate once, as in the reference).

Errors: shape and capacity violations raise ValueError before any launch
(the reference's ``ensure!``); a non-zero status from the library raises
pegainfer_amd._lib.KernelError carrying pegainfer_kernels_last_error().
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum

import torch

from . import _lib

KIMI_K2_HIDDEN = 7168
KIMI_K2_EXPERT_INTERMEDIATE = 2048
KIMI_K2_SHARED_GATE_UP = 2 * KIMI_K2_EXPERT_INTERMEDIATE
KIMI_K2_ROUTED_EXPERTS = 384
KIMI_K2_EP_WORLD = 8
KIMI_K2_LOCAL_EXPERTS = KIMI_K2_ROUTED_EXPERTS // KIMI_K2_EP_WORLD
KIMI_K2_TOPK = 8
KIMI_K2_INT4_GROUP_SIZE = 32
KIMI_K2_ROUTER_SCALE = 2.827  # pegainfer-kernels/src/ops/kimi_k2/router.rs:18
KIMI_MARLIN_MAX_BLOCK_SIZE = 64  # pegainfer-kimi-k2/src/runner/worker.rs:91


def _ensure(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int:
    if t is None:
        return 0
    _ensure(t.is_cuda, "tensor must live on the GPU")
    _ensure(t.is_contiguous(), "tensor must be contiguous")
    return t.data_ptr()


def _is_bf16(t: torch.Tensor) -> bool:
    return t.dtype in (torch.bfloat16, torch.uint16, torch.int16)


# --------------------------------------------------------------------------
# Checkpoint contract (experts.rs:149-401)
# --------------------------------------------------------------------------
class KimiInt4ExpertRole(enum.Enum):
    W1Gate = "w1_gate"
    W3Up = "w3_up"
    W2Down = "w2_down"

    def expected_shape(self) -> "KimiInt4LogicalShape":
        if self is KimiInt4ExpertRole.W2Down:
            return KimiInt4LogicalShape(out_dim=KIMI_K2_HIDDEN, in_dim=KIMI_K2_EXPERT_INTERMEDIATE)
        return KimiInt4LogicalShape(out_dim=KIMI_K2_EXPERT_INTERMEDIATE, in_dim=KIMI_K2_HIDDEN)

    @property
    def label(self) -> str:
        return self.value


class KimiInt4NibbleOrder(enum.Enum):
    LowThenHigh = "low_then_high"
    HighThenLow = "high_then_low"


@dataclasses.dataclass(frozen=True)
class KimiInt4LogicalShape:
    out_dim: int
    in_dim: int


@dataclasses.dataclass(frozen=True)
class KimiInt4TensorShape:
    experts: int
    rows: int
    cols: int

    def elements(self) -> int:
        return self.experts * self.rows * self.cols


@dataclasses.dataclass(frozen=True)
class KimiInt4WeightManifest:
    role: KimiInt4ExpertRole
    global_experts: int
    local_experts: int
    local_expert_offset: int
    logical_shape: KimiInt4LogicalShape
    packed_shape: KimiInt4TensorShape
    scale_shape: KimiInt4TensorShape
    group_size: int
    nibble_order: KimiInt4NibbleOrder

    @classmethod
    def ep8(cls, role: KimiInt4ExpertRole, ep_rank: int,
            nibble_order: KimiInt4NibbleOrder) -> "KimiInt4WeightManifest":
        ls = role.expected_shape()
        return cls(
            role=role, global_experts=KIMI_K2_ROUTED_EXPERTS,
            local_experts=KIMI_K2_LOCAL_EXPERTS,
            local_expert_offset=ep_rank * KIMI_K2_LOCAL_EXPERTS, logical_shape=ls,
            packed_shape=KimiInt4TensorShape(KIMI_K2_LOCAL_EXPERTS, ls.out_dim, (ls.in_dim + 1) // 2),
            scale_shape=KimiInt4TensorShape(KIMI_K2_LOCAL_EXPERTS, ls.out_dim,
                                            ls.in_dim // KIMI_K2_INT4_GROUP_SIZE),
            group_size=KIMI_K2_INT4_GROUP_SIZE, nibble_order=nibble_order)

    def validate(self) -> None:
        _ensure(self.global_experts == KIMI_K2_ROUTED_EXPERTS,
                f"Kimi-K2 routed experts must be {KIMI_K2_ROUTED_EXPERTS}, got {self.global_experts}")
        _ensure(self.local_experts == KIMI_K2_LOCAL_EXPERTS,
                f"Kimi-K2 EP8 rank must own {KIMI_K2_LOCAL_EXPERTS} local experts, got {self.local_experts}")
        _ensure(self.local_expert_offset + self.local_experts <= self.global_experts,
                "local expert range exceeds the global experts")
        _ensure(self.logical_shape == self.role.expected_shape(),
                f"{self.role.label} logical shape must be {self.role.expected_shape()}")
        _ensure(self.group_size == KIMI_K2_INT4_GROUP_SIZE,
                f"Kimi-K2 INT4 group size must be {KIMI_K2_INT4_GROUP_SIZE}, got {self.group_size}")
        _ensure(self.logical_shape.in_dim % self.group_size == 0,
                "input dim must be divisible by the group size")
        _ensure(self.packed_shape == KimiInt4TensorShape(
            self.local_experts, self.logical_shape.out_dim, (self.logical_shape.in_dim + 1) // 2),
            f"{self.role.label} weight_packed shape mismatch")
        _ensure(self.scale_shape == KimiInt4TensorShape(
            self.local_experts, self.logical_shape.out_dim,
            self.logical_shape.in_dim // self.group_size),
            f"{self.role.label} weight_scale shape mismatch")

    def marlin_packed_u32_elements(self) -> int:
        return self.local_experts * (self.logical_shape.in_dim // 16) * (self.logical_shape.out_dim * 2)


def validate_marlin_block_size(block_size: int) -> None:
    _ensure(block_size == 8 or (16 <= block_size <= 64 and block_size % 16 == 0),
            f"Kimi Marlin block_size must be 8 or a multiple of 16 in [16, 64], got {block_size}")


def marlin_padded_route_capacity(active_tokens: int, block_size: int, topk: int = KIMI_K2_TOPK,
                                 local_experts: int = KIMI_K2_LOCAL_EXPERTS) -> int:
    """routes + E*(bs-1) (experts.rs:1500-1511)."""
    validate_marlin_block_size(block_size)
    return active_tokens * topk + local_experts * (block_size - 1)


def kimi_marlin_block_size(active_tokens: int, topk: int = KIMI_K2_TOPK,
                           local_experts: int = KIMI_K2_LOCAL_EXPERTS) -> int:
    """Smallest block size whose expected routes per expert block stay below
    0.9 (pegainfer-kimi-k2/src/runner/worker/runtime.rs:99-109, f32 math)."""
    import numpy as np
    for bs in (8, 16, 32, 48, KIMI_MARLIN_MAX_BLOCK_SIZE):
        per_block = (np.float32(active_tokens) * np.float32(topk) / np.float32(local_experts)
                     / np.float32(bs))
        if per_block < np.float32(0.9):
            return bs
    return KIMI_MARLIN_MAX_BLOCK_SIZE


# --------------------------------------------------------------------------
# Routing workspace / permutation (experts.rs:508-600, 708-848)
# --------------------------------------------------------------------------
class KimiMarlinRouteWorkspace:
    """Device buffers of the token -> expert permutation, sized once for
    `max_active_tokens` (allocation happens here, never per step)."""

    def __init__(self, max_active_tokens: int, block_size: int, *, device="cuda",
                 topk: int = KIMI_K2_TOPK, local_experts: int = KIMI_K2_LOCAL_EXPERTS):
        _ensure(max_active_tokens > 0, "Kimi Marlin route max_active_tokens must be positive")
        validate_marlin_block_size(block_size)
        self.max_active_tokens = max_active_tokens
        self.block_size = block_size
        self.topk = topk
        self.local_experts = local_experts
        self.max_padded_tokens = marlin_padded_route_capacity(max_active_tokens, block_size, topk,
                                                              local_experts)
        self.max_m_blocks = -(-self.max_padded_tokens // block_size)
        i32 = dict(dtype=torch.int32, device=device)
        self.sorted_token_ids = torch.zeros(self.max_padded_tokens, **i32)
        self.expert_ids = torch.zeros(self.max_m_blocks, **i32)
        self.num_tokens_post_padded = torch.zeros(1, **i32)
        # u32 on device; torch has no general uint32 arithmetic, so int32 storage
        self.expert_offsets = torch.zeros(local_experts + 1, **i32)
        self.expert_cursor = torch.zeros(local_experts, **i32)


@dataclasses.dataclass
class KimiMarlinRouting:
    batch_size: int
    active_tokens: int
    route_elems: int
    global_expert_start: int
    block_size: int
    max_padded_tokens: int
    max_m_blocks: int
    topk: int
    local_experts: int
    sorted_token_ids: torch.Tensor
    expert_ids: torch.Tensor
    num_tokens_post_padded: torch.Tensor

    def manifest_attrs(self) -> dict:
        """Attributes of the reference's KernelCall manifest (experts.rs:727-764)."""
        return {"batch_size": str(self.batch_size), "active_tokens": str(self.active_tokens),
                "route_elems": str(self.route_elems), "topk": str(self.topk),
                "local_experts": str(self.local_experts),
                "global_expert_start": str(self.global_expert_start),
                "block_size": str(self.block_size), "sentinel_token_id": str(self.route_elems),
                "device_resident_metadata": "true", "decode_step_allocation": "forbidden",
                "decode_step_d2h": "forbidden"}


def moe_align_block_size(workspace: KimiMarlinRouteWorkspace, topk_idx: torch.Tensor,
                         batch_size: int, active_tokens: int,
                         global_expert_start: int) -> KimiMarlinRouting:
    """Token -> expert permutation (experts.rs:767-848).  Kimi shapes go through
    the reference symbol; other expert counts / top-k through the general one."""
    ws = workspace
    _ensure(active_tokens > 0, "Kimi Marlin route active_tokens must be positive")
    _ensure(active_tokens <= ws.max_active_tokens,
            f"active_tokens {active_tokens} exceeds Kimi Marlin route workspace capacity "
            f"{ws.max_active_tokens}")
    _ensure(batch_size > 0, "batch_size must be > 0")
    _ensure(active_tokens >= batch_size,
            f"active_tokens {active_tokens} must cover batch_size {batch_size}")
    route_elems = active_tokens * ws.topk
    _ensure(topk_idx.dtype == torch.int32, "topk_idx must be int32")
    _ensure(topk_idx.numel() >= route_elems,
            f"topk_idx len must cover active_tokens * topk: have {topk_idx.numel()}, need {route_elems}")
    kimi = ws.topk == KIMI_K2_TOPK and ws.local_experts == KIMI_K2_LOCAL_EXPERTS
    if kimi:
        _ensure(global_expert_start + KIMI_K2_LOCAL_EXPERTS <= KIMI_K2_ROUTED_EXPERTS,
                "global expert range exceeds the routed experts")
    name = "kimi_moe_marlin_align_block_size_cuda" if kimi else "pega_moe_align_block_size"
    _lib.call(name, _ptr(topk_idx), _ptr(ws.sorted_token_ids), _ptr(ws.expert_ids),
              _ptr(ws.num_tokens_post_padded), _ptr(ws.expert_offsets), _ptr(ws.expert_cursor),
              active_tokens, ws.topk, global_expert_start, ws.local_experts, ws.block_size,
              ws.max_padded_tokens, ws.max_m_blocks, _stream())
    return KimiMarlinRouting(batch_size, active_tokens, route_elems, global_expert_start,
                             ws.block_size, ws.max_padded_tokens, ws.max_m_blocks, ws.topk,
                             ws.local_experts, ws.sorted_token_ids, ws.expert_ids,
                             ws.num_tokens_post_padded)


kimi_moe_marlin_align_block_size = moe_align_block_size


def kimi_deepep_build_marlin_routing_on_stream(workspace: KimiMarlinRouteWorkspace,
                                               psum_expert: torch.Tensor, expert_alignment: int,
                                               expanded_capacity: int) -> KimiMarlinRouting:
    """Routing metadata for an expert-major buffer (experts.rs:1250-1325)."""
    ws = workspace
    _ensure(expert_alignment > 0, "deepep expert_alignment must be positive")
    _ensure(expert_alignment % ws.block_size == 0,
            f"deepep expert_alignment {expert_alignment} must be a multiple of Marlin block_size "
            f"{ws.block_size}")
    _ensure(psum_expert.numel() > ws.local_experts,
            f"psum_expert len must be >= {ws.local_experts + 1}")
    _ensure(expanded_capacity <= ws.max_padded_tokens,
            f"deepep expanded_capacity {expanded_capacity} exceeds workspace max_padded_tokens "
            f"{ws.max_padded_tokens}")
    tight_m_blocks = -(-expanded_capacity // ws.block_size)
    _lib.call("kimi_deepep_build_marlin_routing_on_stream", _ptr(psum_expert),
              _ptr(ws.sorted_token_ids), _ptr(ws.expert_ids), _ptr(ws.num_tokens_post_padded),
              ws.local_experts, expert_alignment, ws.block_size, expanded_capacity,
              tight_m_blocks, _stream())
    return KimiMarlinRouting(expanded_capacity, expanded_capacity, expanded_capacity, 0,
                             ws.block_size, expanded_capacity, tight_m_blocks, 1,
                             ws.local_experts, ws.sorted_token_ids, ws.expert_ids,
                             ws.num_tokens_post_padded)


# --------------------------------------------------------------------------
# Weight packages (experts.rs:403-506, 850-1022)
# --------------------------------------------------------------------------
@dataclasses.dataclass
class MarlinInt4Weight:
    """One projection in the device layout: packed [E, K/16, 2N] u32 (as
    uint8 bytes) and permuted scales [E, K/32, N] bf16."""
    local_experts: int
    in_dim: int
    out_dim: int
    weight_packed_uint4b8: torch.Tensor
    weight_scale_permuted: torch.Tensor
    group_size: int = KIMI_K2_INT4_GROUP_SIZE

    def validate(self) -> None:
        _ensure(self.group_size == KIMI_K2_INT4_GROUP_SIZE, "group size must be 32")
        _ensure(self.weight_packed_uint4b8.numel() * self.weight_packed_uint4b8.element_size()
                == self.local_experts * self.out_dim * self.in_dim // 2,
                "Marlin uint4b8 packed size mismatch")
        _ensure(self.weight_scale_permuted.numel()
                == self.local_experts * self.out_dim * (self.in_dim // self.group_size),
                "Marlin permuted scale size mismatch")


def _repack_one(ckpt_packed: torch.Tensor, ckpt_scale: torch.Tensor, local_experts: int,
                in_dim: int, out_dim: int, kimi: bool) -> MarlinInt4Weight:
    _ensure(ckpt_packed.numel() * ckpt_packed.element_size() == local_experts * out_dim * in_dim // 2,
            "checkpoint packed size mismatch")
    _ensure(ckpt_scale.numel() == local_experts * out_dim * (in_dim // KIMI_K2_INT4_GROUP_SIZE),
            "checkpoint scale size mismatch")
    packed = torch.empty(local_experts * out_dim * in_dim // 2, dtype=torch.uint8,
                         device=ckpt_packed.device)
    scale = torch.empty(ckpt_scale.numel(), dtype=torch.bfloat16, device=ckpt_scale.device)
    wname = "kimi_marlin_int4_reorder_weight_cuda" if kimi else "pega_marlin_int4_reorder_weight"
    sname = "kimi_marlin_int4_reorder_scale_cuda" if kimi else "pega_marlin_int4_reorder_scale"
    _lib.call(wname, _ptr(ckpt_packed), _ptr(packed), in_dim, out_dim, local_experts,
              KIMI_K2_INT4_GROUP_SIZE, _stream())
    _lib.call(sname, _ptr(ckpt_scale), _ptr(scale), in_dim, out_dim, local_experts,
              KIMI_K2_INT4_GROUP_SIZE, _stream())
    return MarlinInt4Weight(local_experts, in_dim, out_dim, packed, scale)


def kimi_marlin_int4_reorder(ckpt_packed: torch.Tensor, ckpt_scale: torch.Tensor,
                             manifest: KimiInt4WeightManifest) -> MarlinInt4Weight:
    """Checkpoint -> device layout for one Kimi projection (experts.rs:850-951).
    Load-time only: allocates the package."""
    manifest.validate()
    _ensure(manifest.nibble_order is KimiInt4NibbleOrder.LowThenHigh,
            "Marlin repack expects low-then-high offset-binary INT4")
    ls = manifest.logical_shape
    return _repack_one(ckpt_packed, ckpt_scale, manifest.local_experts, ls.in_dim, ls.out_dim,
                       kimi=True)


def marlin_int4_reorder(ckpt_packed: torch.Tensor, ckpt_scale: torch.Tensor, local_experts: int,
                        in_dim: int, out_dim: int) -> MarlinInt4Weight:
    """Shape-general checkpoint -> device layout (any expert count)."""
    return _repack_one(ckpt_packed, ckpt_scale, local_experts, in_dim, out_dim, kimi=False)


def marlin_int4_fuse_w13(gate: MarlinInt4Weight, up: MarlinInt4Weight) -> MarlinInt4Weight:
    """Concatenate gate || up per k-tile row and per group row (experts.rs:953-1022)."""
    _ensure((gate.local_experts, gate.in_dim, gate.out_dim) == (up.local_experts, up.in_dim, up.out_dim),
            "Marlin W13 fuse requires matching shapes")
    gate.validate()
    up.validate()
    w = torch.empty(gate.weight_packed_uint4b8.numel() * 2, dtype=torch.uint8,
                    device=gate.weight_packed_uint4b8.device)
    s = torch.empty(gate.weight_scale_permuted.numel() * 2, dtype=torch.bfloat16,
                    device=gate.weight_scale_permuted.device)
    kimi = gate.local_experts == KIMI_K2_LOCAL_EXPERTS
    name = "kimi_marlin_int4_fuse_w13_cuda" if kimi else "pega_marlin_int4_fuse_w13"
    _lib.call(name, _ptr(gate.weight_packed_uint4b8), _ptr(up.weight_packed_uint4b8), _ptr(w),
              _ptr(gate.weight_scale_permuted), _ptr(up.weight_scale_permuted), _ptr(s),
              gate.in_dim, gate.out_dim, gate.local_experts, KIMI_K2_INT4_GROUP_SIZE, _stream())
    return MarlinInt4Weight(gate.local_experts, gate.in_dim, 2 * gate.out_dim, w, s)


# --------------------------------------------------------------------------
# Grouped GEMM (experts.rs:602-706, 1024-1131, 1403-1473)
# --------------------------------------------------------------------------
class KimiMarlinWna16Workspace:
    """locks = (max_size_n/64) * max_m_blocks i32, c_tmp = max_size_n * max_padded
    f32 (x2 for block size 8), as in experts.rs:612-652; `extra_splits` multiplies
    c_tmp so that the shape-general entry can split K across workgroups."""

    def __init__(self, max_m_blocks: int, max_size_n: int, block_size: int, *, device="cuda",
                 extra_splits: int = 1):
        validate_marlin_block_size(block_size)
        _ensure(max_m_blocks > 0, "Kimi Marlin WNA16 max_m_blocks must be > 0")
        _ensure(max_size_n % 64 == 0, "max_size_n must be divisible by 64")
        self.max_m_blocks = max_m_blocks
        self.max_size_n = max_size_n
        self.block_size = block_size
        self.max_padded_tokens = max_m_blocks * block_size
        self.locks = torch.zeros(max(1, (max_size_n // 64) * max_m_blocks), dtype=torch.int32,
                                 device=device)
        c_tmp = max_size_n * self.max_padded_tokens * (2 if block_size == 8 else 1)
        c_tmp *= max(1, extra_splits)
        self.c_tmp = torch.zeros(max(1, c_tmp), dtype=torch.float32, device=device)


def wna16_gemm(workspace: KimiMarlinWna16Workspace, routing: KimiMarlinRouting,
               input: torch.Tensor, weight: MarlinInt4Weight, topk_weight: torch.Tensor,
               output: torch.Tensor, *, top_k: int, mul_topk_weights: bool, size_m: int) -> None:
    """C[sorted_id] = bf16(A[sorted_id / top_k] . dequant(W[expert]))  (optionally
    times bf16(topk_weight[sorted_id])).  Rows not routed here are left as they are."""
    size_n, size_k = weight.out_dim, weight.in_dim
    _ensure(workspace.block_size == routing.block_size,
            f"Kimi Marlin WNA16 workspace block_size {workspace.block_size} must match routing "
            f"{routing.block_size}")
    _ensure(routing.max_m_blocks <= workspace.max_m_blocks, "workspace max_m_blocks below routing")
    _ensure(size_n <= workspace.max_size_n and size_n % 64 == 0,
            f"size_n {size_n} exceeds workspace max {workspace.max_size_n} or is not divisible by 64")
    _ensure(input.numel() >= size_m * size_k, "input too small")
    _ensure(output.numel() >= size_m * top_k * size_n, "output too small")
    _ensure(topk_weight.dtype == torch.float32, "topk_weight must be float32")
    _ensure(_is_bf16(input) and _is_bf16(output), "input/output must be bf16")
    weight.validate()
    kimi = weight.local_experts == KIMI_K2_LOCAL_EXPERTS
    if kimi:
        _lib.call("kimi_marlin_wna16_gemm_cuda", _ptr(input), _ptr(output), _ptr(workspace.c_tmp),
                  _ptr(weight.weight_packed_uint4b8), _ptr(weight.weight_scale_permuted),
                  _ptr(workspace.locks), _ptr(routing.sorted_token_ids), _ptr(routing.expert_ids),
                  _ptr(routing.num_tokens_post_padded), _ptr(topk_weight), workspace.locks.numel(),
                  routing.max_padded_tokens, routing.block_size, top_k, bool(mul_topk_weights),
                  size_m, size_n, size_k, weight.local_experts, KIMI_K2_INT4_GROUP_SIZE, 0,
                  _stream())
    else:
        _lib.call("pega_wna16_gemm", _ptr(input), _ptr(output), _ptr(workspace.c_tmp),
                  workspace.c_tmp.numel(), _ptr(weight.weight_packed_uint4b8),
                  _ptr(weight.weight_scale_permuted), _ptr(workspace.locks),
                  workspace.locks.numel(), _ptr(routing.sorted_token_ids),
                  _ptr(routing.expert_ids), _ptr(routing.num_tokens_post_padded),
                  _ptr(topk_weight), routing.max_padded_tokens, routing.block_size, top_k,
                  bool(mul_topk_weights), size_m, size_n, size_k, weight.local_experts,
                  KIMI_K2_INT4_GROUP_SIZE, 0, _stream())


def wna16_w13_swiglu(workspace: KimiMarlinWna16Workspace, routing: KimiMarlinRouting,
                     input: torch.Tensor, weight: MarlinInt4Weight, act: torch.Tensor, *,
                     top_k: int, size_m: int, split_k: bool = True) -> None:
    """act[sorted_id] = SwiGLU(bf16(A[sorted_id / top_k] . dequant(W13[expert]))) in one
    call, routed rows only.  Block sizes 8/16: when too few workgroups would fill the GPU,
    K is split across workgroups and the partials (the workspace's c_tmp) are summed by the
    SwiGLU kernel; otherwise (or with split_k=False) a gate tile and its up tile share a
    workgroup with SwiGLU in the epilogue.  32/48/64: the tile GEMM with a SwiGLU epilogue."""
    inter = weight.out_dim // 2
    _ensure(workspace.block_size == routing.block_size, "workspace / routing block size differ")
    _ensure(2 * inter <= workspace.max_size_n, "W13 width exceeds the workspace")
    _ensure(act.dtype == torch.bfloat16 and act.numel() >= size_m * top_k * inter,
            "act must be bf16 [size_m * top_k, inter]")
    _lib.call("pega_wna16_w13_swiglu", _ptr(input), _ptr(act),
              _ptr(workspace.c_tmp) if split_k else None,
              workspace.c_tmp.numel() if split_k else 0, _ptr(weight.weight_packed_uint4b8),
              _ptr(weight.weight_scale_permuted), _ptr(routing.sorted_token_ids),
              _ptr(routing.expert_ids), _ptr(routing.num_tokens_post_padded),
              routing.sorted_token_ids.numel(), routing.block_size, top_k, size_m, inter,
              weight.in_dim, weight.local_experts, 32, 0, _stream())


def wna16_problem(routing: KimiMarlinRouting, input: torch.Tensor, weight: MarlinInt4Weight, *,
                  top_k: int, size_m: int, output: torch.Tensor = None, act: torch.Tensor = None,
                  topk_weight: torch.Tensor = None,
                  mul_topk_weights: bool = False) -> "_lib.Wna16Problem":
    """One prefill-size GEMM for wna16_prefill_pair: as wna16_gemm (output) or
    wna16_w13_swiglu (act).  The struct holds raw pointers: the tensors must
    stay alive until the launch."""
    _ensure((output is None) != (act is None), "give exactly one of output and act")
    _ensure(routing.block_size > 16, f"block size {routing.block_size}: the pair launch runs "
            "the prefill tile kernel (block sizes 32, 48, 64)")
    size_n, size_k = weight.out_dim, weight.in_dim
    _ensure(_is_bf16(input) and input.numel() >= size_m * size_k, "input must be bf16 [size_m, K]")
    if act is not None:
        _ensure(not mul_topk_weights, "the SwiGLU epilogue applies no top-k weight")
        _ensure(_is_bf16(act) and act.numel() >= size_m * top_k * (size_n // 2),
                "act must be bf16 [size_m * top_k, inter]")
    else:
        _ensure(_is_bf16(output) and output.numel() >= size_m * top_k * size_n,
                "output must be bf16 [size_m * top_k, N]")
    if mul_topk_weights:
        _ensure(topk_weight is not None and topk_weight.dtype == torch.float32,
                "mul_topk_weights needs float32 topk weights")
    weight.validate()
    return _lib.Wna16Problem(
        _ptr(input), _ptr(output) if output is not None else None,
        _ptr(act) if act is not None else None, _ptr(weight.weight_packed_uint4b8),
        _ptr(weight.weight_scale_permuted), _ptr(routing.sorted_token_ids),
        _ptr(routing.expert_ids), _ptr(routing.num_tokens_post_padded),
        _ptr(topk_weight) if topk_weight is not None else None,
        routing.sorted_token_ids.numel(), routing.block_size, top_k, int(bool(mul_topk_weights)),
        size_m, size_n, size_k, weight.local_experts, KIMI_K2_INT4_GROUP_SIZE)


def wna16_prefill_pair(first: "_lib.Wna16Problem", second: "_lib.Wna16Problem") -> None:
    """Both GEMMs in one launch (the first problem's workgroups dispatched
    first); each output has the bits of its own single launch."""
    _lib.call("pega_wna16_prefill_pair", ctypes.byref(first), ctypes.byref(second), _stream())


def kimi_marlin_wna16_expanded_w13_gemm(workspace, routing, input, weight, topk_weight,
                                        output_w13):
    """W13 over the DeepEP expanded (expert-major) buffer: top_k = 1, no weight
    multiply, size_m = the expanded capacity (experts.rs:1328-1360).  `routing` comes
    from kimi_deepep_build_marlin_routing_on_stream: identity ids for real rows, the
    capacity sentinel for pad rows, read on device up to num_tokens_post_padded."""
    _ensure(topk_weight.numel() >= routing.route_elems,
            f"topk_weight len must cover {routing.route_elems}, got {topk_weight.numel()}")
    wna16_gemm(workspace, routing, input, weight, topk_weight, output_w13, top_k=1,
               mul_topk_weights=False, size_m=routing.active_tokens)


def kimi_marlin_wna16_expanded_w2_gemm(workspace, routing, input, weight, topk_weight, output):
    """W2 over the DeepEP expanded buffer: top_k = 1, one bf16 top-k weight per
    expert-major row, size_m = route_elems (experts.rs:1364-1401)."""
    _ensure(topk_weight.numel() >= routing.route_elems,
            f"topk_weight len must cover {routing.route_elems}, got {topk_weight.numel()}")
    wna16_gemm(workspace, routing, input, weight, topk_weight, output, top_k=1,
               mul_topk_weights=True, size_m=routing.route_elems)


def kimi_marlin_wna16_w13_gemm(workspace, routing, input, weight, topk_weight, output_w13):
    """W13 call: top_k = routing.topk, no weight multiply, size_m = active tokens
    (experts.rs:1024-1080)."""
    _ensure(output_w13.numel() >= routing.route_elems * weight.out_dim,
            "marlin_w13 output must cover route_elems rows")
    wna16_gemm(workspace, routing, input, weight, topk_weight, output_w13, top_k=routing.topk,
               mul_topk_weights=False, size_m=routing.active_tokens)


def kimi_marlin_wna16_w2_gemm(workspace, routing, input, weight, topk_weight, output):
    """W2 call: top_k = 1, multiply by bf16(topk weight), size_m = route_elems
    (experts.rs:1082-1131)."""
    wna16_gemm(workspace, routing, input, weight, topk_weight, output, top_k=1,
               mul_topk_weights=True, size_m=routing.route_elems)


# --------------------------------------------------------------------------
# Elementwise stages (experts.rs:27-147, 1133-1240)
# --------------------------------------------------------------------------
def kimi_marlin_w13_swiglu(w13: torch.Tensor, output: torch.Tensor, rows: int, inter: int) -> None:
    _ensure(w13.numel() >= rows * 2 * inter and output.numel() >= rows * inter,
            "Kimi Marlin SwiGLU size mismatch")
    _lib.call("kimi_marlin_w13_swiglu_cuda", _ptr(w13), _ptr(output), rows, inter, _stream())


def kimi_marlin_w13_swiglu_expanded(w13: torch.Tensor, num_tokens_post_padded: torch.Tensor,
                                    output: torch.Tensor, max_rows: int, inter: int) -> None:
    _ensure(num_tokens_post_padded.numel() >= 1,
            "num_tokens_post_padded must have at least 1 element")
    _lib.call("kimi_marlin_w13_swiglu_expanded_cuda", _ptr(w13), _ptr(output),
              _ptr(num_tokens_post_padded), max_rows, inter, 0, _stream())


def kimi_marlin_sum_topk_rows_f32(route_output: torch.Tensor, active_tokens: int,
                                  out: torch.Tensor, topk: int, hidden: int) -> None:
    _ensure(route_output.numel() >= active_tokens * topk * hidden, "route_output too small")
    _ensure(out.numel() >= active_tokens * hidden, "marlin_sum_topk output too small")
    _lib.call("kimi_marlin_sum_topk_rows_f32_cuda", _ptr(route_output), _ptr(out),
              active_tokens, topk, hidden, _stream())


def weighted_topk_sum_f32(route_output: torch.Tensor, topk_weight: torch.Tensor,
                          active_tokens: int, out: torch.Tensor, topk: int, hidden: int) -> None:
    _lib.call("pega_weighted_topk_sum_f32", _ptr(route_output), _ptr(topk_weight), _ptr(out),
              active_tokens, topk, hidden, _stream())


def moe_combine_local_f32(route_output: torch.Tensor, topk_idx: torch.Tensor,
                          topk_weight, active_tokens: int, out: torch.Tensor, topk: int,
                          hidden: int, global_start: int, local_experts: int) -> None:
    """Top-k combine over local routes only (rows of other routes are not read).
    `topk_weight` None: plain sum; a tensor: fmaf chain with those weights."""
    _ensure(route_output.numel() >= active_tokens * topk * hidden, "route_output too small")
    _ensure(out.numel() >= active_tokens * hidden, "combine output too small")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= active_tokens * topk,
            "topk_idx must be int32 [tokens, topk]")
    _lib.call("pega_moe_combine_local_f32", _ptr(route_output), _ptr(topk_idx),
              None if topk_weight is None else _ptr(topk_weight), _ptr(out), active_tokens,
              topk, hidden, global_start, local_experts, _stream())


def kimi_residual_add_scaled_f32(hidden, projected, routed_f32, scale, out) -> None:
    n = hidden.numel()
    _ensure(projected.numel() == n and out.numel() == n, "residual_add_scaled_f32 size mismatch")
    _ensure(routed_f32.numel() >= n, "routed_f32 too small")
    _lib.call("kimi_residual_add_scaled_f32_cuda", _ptr(hidden), _ptr(projected),
              _ptr(routed_f32), float(scale), _ptr(out), n, _stream())


def kimi_residual_add_scaled_bf16(hidden, projected, routed, scale, out) -> None:
    n = hidden.numel()
    _ensure(projected.numel() == n and out.numel() == n, "residual_add_scaled_bf16 size mismatch")
    _ensure(routed.numel() >= n, "routed too small")
    _lib.call("kimi_residual_add_scaled_bf16_cuda", _ptr(hidden), _ptr(projected), _ptr(routed),
              float(scale), _ptr(out), n, _stream())


def kimi_add_f32_bf16_to_bf16(a, b, out) -> None:
    n = b.numel()
    _ensure(a.numel() >= n and out.numel() == n, "Kimi f32 add size mismatch")
    _lib.call("kimi_add_f32_bf16_to_bf16_cuda", _ptr(a), _ptr(b), _ptr(out), n, _stream())


def f32_to_bf16(x: torch.Tensor, out: torch.Tensor) -> None:
    """out = bf16(x) (f32_to_bf16_hidden_into, pegainfer-kernels/src/ops/elementwise.rs:579-603)."""
    n = out.numel()
    _ensure(x.dtype == torch.float32 and x.numel() >= n,
            f"f32 input len {x.numel()} < bf16 output len {n}")
    _ensure(_is_bf16(out), "f32_to_bf16 output must be bf16")
    _lib.call("f32_to_bf16_cuda", _ptr(x), _ptr(out), n, _stream())


def add_bf16(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor) -> None:
    """out = bf16(a + b) over bf16 tensors (add_batch_into, elementwise.rs:14-40)."""
    _ensure(a.numel() == b.numel() == out.numel(), "add: shapes differ")
    _ensure(_is_bf16(a) and _is_bf16(b) and _is_bf16(out), "add operands must be bf16")
    _lib.call("add_cuda", _ptr(a), _ptr(b), _ptr(out), out.numel(), _stream())


def moe_join_routed_shared(routed_f32: torch.Tensor, shared: torch.Tensor,
                           out: torch.Tensor) -> None:
    """DeepSeek-V2-Lite routed + shared join, rounded as the reference does it:
    out = bf16(f(bf16(routed)) + f(shared)) (nccl_backend.rs:544-545 then
    runtime/moe.rs:656), in one launch."""
    n = out.numel()
    _ensure(routed_f32.dtype == torch.float32 and routed_f32.numel() >= n, "routed too small")
    _ensure(shared.numel() == n and _is_bf16(shared) and _is_bf16(out),
            "shared / out must be bf16 of the same size")
    _lib.call("pega_moe_join_routed_shared_bf16", _ptr(routed_f32), _ptr(shared), _ptr(out), n,
              _stream())


def moe_combine_join(route_output: torch.Tensor, topk_idx: torch.Tensor, topk_weight,
                     shared: torch.Tensor, out: torch.Tensor, active_tokens: int, topk: int,
                     hidden: int, global_start: int, local_experts: int) -> None:
    """moe_combine_local_f32 then moe_join_routed_shared in one launch (no fp32 rows in
    between), for a layer whose routed sum needs no cross-GPU reduction before the
    join: out = bf16(f(bf16(combine)) + f(shared)), the same bits as the two calls."""
    _ensure(route_output.numel() >= active_tokens * topk * hidden and _is_bf16(route_output),
            "route_output must be bf16 [tokens * topk, hidden]")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= active_tokens * topk,
            "topk_idx must be int32 [tokens, topk]")
    _ensure(topk_weight is None or (topk_weight.dtype == torch.float32 and
                                    topk_weight.numel() >= active_tokens * topk),
            "topk_weight must be float32 [tokens, topk]")
    _ensure(_is_bf16(shared) and _is_bf16(out) and shared.numel() >= active_tokens * hidden
            and out.numel() >= active_tokens * hidden, "shared / out must be bf16 [tokens, hidden]")
    _lib.call("pega_moe_combine_join_bf16", _ptr(route_output), _ptr(topk_idx),
              None if topk_weight is None else _ptr(topk_weight), _ptr(shared), _ptr(out),
              active_tokens, topk, hidden, global_start, local_experts, _stream())


# --------------------------------------------------------------------------
# Dense bf16 GEMM (the shared expert's projections)
# --------------------------------------------------------------------------
def gemm_graphsafe(w: torch.Tensor, x: torch.Tensor, y: torch.Tensor) -> None:
    """Y[n][m] = bf16(sum_k W[m][k] * X[n][k]) with fp32 accumulation: W [M, K]
    (a DeviceMatrix, rows = output features), X [N, K], Y [N, M], all bf16.
    Mirrors typed_ops.rs:296-344 (gemm_dm_typed_to_hs_graphsafe /
    gemm_dm_hs_to_typed_graphsafe -> gemm_graphsafe_cuda)."""
    _ensure(_is_bf16(w) and _is_bf16(x) and _is_bf16(y), "dense GEMM operands must be bf16")
    _ensure(w.dim() == 2 and x.dim() == 2 and y.dim() == 2, "dense GEMM operands must be 2-D")
    _ensure(w.is_contiguous() and x.is_contiguous() and y.is_contiguous(),
            "dense GEMM operands must be contiguous")
    M, K = w.shape
    N = x.shape[0]
    _ensure(x.shape[1] == K, f"DM GEMM weight cols={K} must match input dim {x.shape[1]}")
    _ensure(tuple(y.shape) == (N, M),
            f"DM GEMM shape mismatch: w.rows={M}, y={tuple(y.shape)}, x.seq={N}")
    _lib.call("gemm_graphsafe_cuda", _ptr(w), _ptr(x), _ptr(y), M, N, K, _stream())


def dense_w13_swiglu(w13: torch.Tensor, x: torch.Tensor, act: torch.Tensor) -> None:
    """act = SwiGLU(bf16(X * W13^T)) in one launch: W13 [2I, K] bf16 (gate rows
    first), X [N, K], act [N, I].  The same bits as gemm_graphsafe followed by
    silu_mul_fused_cuda, the pair the reference runs for the shared expert
    (moe_nccl.rs:113-117; csrc/shared/fused_proj.cu:11-31), whose per-element
    formula bf16(f(bf16(silu(g))) * u) is kimi_marlin_w13_swiglu's."""
    _ensure(_is_bf16(w13) and _is_bf16(x) and _is_bf16(act), "dense SwiGLU operands must be bf16")
    _ensure(w13.dim() == 2 and x.dim() == 2 and act.dim() == 2,
            "dense SwiGLU operands must be 2-D")
    _ensure(w13.is_contiguous() and x.is_contiguous() and act.is_contiguous(),
            "dense SwiGLU operands must be contiguous")
    two_i, K = w13.shape
    N = x.shape[0]
    _ensure(two_i % 2 == 0 and x.shape[1] == K, "dense SwiGLU shape mismatch")
    _ensure(tuple(act.shape) == (N, two_i // 2), "dense SwiGLU output shape mismatch")
    _lib.call("pega_dense_w13_swiglu", _ptr(w13), _ptr(x), _ptr(act), two_i // 2, N, K, _stream())


# --------------------------------------------------------------------------
# Routing select
# --------------------------------------------------------------------------
ROUTE_ALIGN_MAX_ROUTES = 4096  # routes the fused select + permutation keeps in one workgroup


def _ensure_router_inputs(logits: torch.Tensor, bias, active_tokens: int, n_experts: int) -> None:
    """The select kernels read active_tokens rows of logits and n_experts biases on the
    device: reject tensors that do not cover them."""
    _ensure(logits.dtype == torch.float32, "logits must be f32")
    _ensure(logits.is_contiguous(), "logits must be contiguous [tokens, n_experts]")
    _ensure(logits.numel() >= active_tokens * n_experts,
            f"logits must cover {active_tokens} rows of {n_experts} experts")
    if bias is not None:
        _ensure(bias.dtype == torch.float32, "bias must be f32")
        _ensure(bias.numel() >= n_experts, f"bias must cover {n_experts} experts")


def kimi_route_align(workspace: KimiMarlinRouteWorkspace, logits: torch.Tensor, bias: torch.Tensor,
                     topk_weight: torch.Tensor, topk_idx: torch.Tensor, active_tokens: int,
                     global_expert_start: int, route_scale: float = 1.0) -> KimiMarlinRouting:
    """The router's select stage and the token -> expert permutation in one launch
    (pega_kimi_route_align): the outputs of kimi_router_select followed by
    moe_align_block_size, bit for bit, for decode batches (at most 4096 routes)."""
    ws = workspace
    n_experts = logits.shape[-1]
    _ensure(active_tokens > 0, "Kimi Marlin route active_tokens must be positive")
    _ensure_router_inputs(logits, bias, active_tokens, n_experts)
    _ensure(active_tokens <= ws.max_active_tokens,
            f"active_tokens {active_tokens} exceeds Kimi Marlin route workspace capacity "
            f"{ws.max_active_tokens}")
    route_elems = active_tokens * ws.topk
    _ensure(route_elems <= ROUTE_ALIGN_MAX_ROUTES,
            f"{route_elems} routes exceed the fused select + permutation's {ROUTE_ALIGN_MAX_ROUTES}")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= route_elems,
            "topk_idx must be int32 covering active_tokens * topk")
    _ensure(topk_weight.dtype == torch.float32 and topk_weight.numel() >= route_elems,
            "topk_weight must be f32 covering active_tokens * topk")
    _lib.call("pega_kimi_route_align", _ptr(logits), _ptr(bias), _ptr(topk_weight), _ptr(topk_idx),
              _ptr(ws.sorted_token_ids), _ptr(ws.expert_ids), _ptr(ws.num_tokens_post_padded),
              _ptr(ws.expert_offsets), _ptr(ws.expert_cursor), active_tokens, n_experts, ws.topk,
              float(route_scale), global_expert_start, ws.local_experts, ws.block_size,
              ws.max_padded_tokens, ws.max_m_blocks, _stream())
    return KimiMarlinRouting(active_tokens, active_tokens, route_elems, global_expert_start,
                             ws.block_size, ws.max_padded_tokens, ws.max_m_blocks, ws.topk,
                             ws.local_experts, ws.sorted_token_ids, ws.expert_ids,
                             ws.num_tokens_post_padded)


def dsv2_route_align(workspace: KimiMarlinRouteWorkspace, logits: torch.Tensor,
                     topk_weight: torch.Tensor, topk_idx: torch.Tensor, tokens: int,
                     global_expert_start: int) -> KimiMarlinRouting:
    """The DeepSeek-V2-Lite router (softmax top-k ordered by expert id) and the
    token -> expert permutation in one launch (pega_dsv2_route_align): the outputs of
    dsv2_router_select followed by moe_align_block_size, bit for bit (at most 4096
    routes)."""
    ws = workspace
    n_experts = logits.shape[-1]
    _ensure(tokens > 0, "tokens must be positive")
    _ensure_router_inputs(logits, None, tokens, n_experts)
    _ensure(tokens <= ws.max_active_tokens,
            f"tokens {tokens} exceed the route workspace capacity {ws.max_active_tokens}")
    route_elems = tokens * ws.topk
    _ensure(route_elems <= ROUTE_ALIGN_MAX_ROUTES,
            f"{route_elems} routes exceed the fused select + permutation's {ROUTE_ALIGN_MAX_ROUTES}")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= route_elems,
            "topk_idx must be int32 covering tokens * topk")
    _ensure(topk_weight.dtype == torch.float32 and topk_weight.numel() >= route_elems,
            "topk_weight must be f32 covering tokens * topk")
    _lib.call("pega_dsv2_route_align", _ptr(logits), _ptr(topk_weight), _ptr(topk_idx),
              _ptr(ws.sorted_token_ids), _ptr(ws.expert_ids), _ptr(ws.num_tokens_post_padded),
              _ptr(ws.expert_offsets), _ptr(ws.expert_cursor), tokens, n_experts, ws.topk,
              global_expert_start, ws.local_experts, ws.block_size, ws.max_padded_tokens,
              ws.max_m_blocks, _stream())
    return KimiMarlinRouting(tokens, tokens, route_elems, global_expert_start, ws.block_size,
                             ws.max_padded_tokens, ws.max_m_blocks, ws.topk, ws.local_experts,
                             ws.sorted_token_ids, ws.expert_ids, ws.num_tokens_post_padded)


def kimi_router_select(logits: torch.Tensor, bias: torch.Tensor, topk_weight: torch.Tensor,
                       topk_idx: torch.Tensor, active_tokens: int, topk: int = KIMI_K2_TOPK,
                       route_scale: float = 1.0) -> None:
    n_experts = logits.shape[-1]
    _ensure_router_inputs(logits, bias, active_tokens, n_experts)
    _ensure(topk_weight.dtype == torch.float32 and topk_weight.numel() >= active_tokens * topk,
            "topk_weight must be f32 covering active_tokens * topk")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= active_tokens * topk,
            "topk_idx must be int32 covering active_tokens * topk")
    _lib.call("pega_kimi_router_select", _ptr(logits), _ptr(bias), _ptr(topk_weight),
              _ptr(topk_idx), active_tokens, n_experts, topk, float(route_scale), _stream())


def kimi_k2_router_noaux_tc(hidden: torch.Tensor, gate_weight: torch.Tensor,
                            e_score_correction_bias: torch.Tensor, logits: torch.Tensor,
                            topk_weight: torch.Tensor, topk_idx: torch.Tensor, active_tokens: int,
                            padded_tokens: int, route_scale: float = 1.0) -> None:
    """The Kimi router in one call (router.rs:182-229 -> kimi_k2_router_noaux_tc_cuda):
    fp32 logits [padded_tokens, 384] = hidden . gate^T, then sigmoid top-8 of
    score + bias with renormalised weights for the first active_tokens rows."""
    n_experts, hidden_dim = gate_weight.shape
    _ensure(_is_bf16(hidden) and _is_bf16(gate_weight), "hidden / gate_weight must be bf16")
    _ensure(hidden.numel() >= padded_tokens * hidden_dim, "hidden must cover padded_tokens rows")
    _ensure(logits.dtype == torch.float32 and logits.numel() >= padded_tokens * n_experts,
            "logits must be f32 [padded_tokens, n_experts]")
    _ensure(e_score_correction_bias.dtype == torch.float32 and
            e_score_correction_bias.numel() >= n_experts, "bias must be f32 [n_experts]")
    _ensure(topk_weight.numel() >= active_tokens * KIMI_K2_TOPK and
            topk_idx.numel() >= active_tokens * KIMI_K2_TOPK, "top-k outputs too small")
    _lib.call("kimi_k2_router_noaux_tc_cuda", _ptr(hidden), _ptr(gate_weight),
              _ptr(e_score_correction_bias), _ptr(logits), _ptr(topk_weight), _ptr(topk_idx),
              active_tokens, padded_tokens, hidden_dim, n_experts, KIMI_K2_TOPK,
              float(route_scale), _stream())


def dsv2_router_select(logits: torch.Tensor, topk_weight: torch.Tensor, topk_idx: torch.Tensor,
                       tokens: int, topk: int = 6) -> None:
    n_experts = logits.shape[-1]
    _ensure_router_inputs(logits, None, tokens, n_experts)
    _ensure(topk_weight.dtype == torch.float32 and topk_weight.numel() >= tokens * topk,
            "topk_weight must be f32 covering tokens * topk")
    _ensure(topk_idx.dtype == torch.int32 and topk_idx.numel() >= tokens * topk,
            "topk_idx must be int32 covering tokens * topk")
    _lib.call("pega_dsv2_router_select", _ptr(logits), _ptr(topk_weight), _ptr(topk_idx),
              tokens, n_experts, topk, _stream())
