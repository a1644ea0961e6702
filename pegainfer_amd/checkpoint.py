"""Routed-expert INT4 weights from a compressed-tensors checkpoint.

One MoE layer's local experts for one EP rank are read out of the safetensors
shards named by ``model.safetensors.index.json`` (or a single
``model.safetensors``).  Every tensor's dtype and shape is checked, the
experts are concatenated expert-major on the host, and the GPU repacks them
into the device layout with W13 fused.  The reference's loader does the same:

* tensor names: ``language_model.model.layers.{L}.mlp.experts.{e}.{proj}.``
  ``weight_packed`` / ``weight_scale``
  (pegainfer-kimi-k2/src/weights/manifest.rs:685-721);
* index parsing: ``weight_map`` name -> shard (manifest.rs:195-206);
* checks: ``weight_packed`` I32 ``[out, in/8]``, ``weight_scale`` BF16
  ``[out, in/32]`` (package.rs:447-484, 765-);
* expert-major concatenation, weight and scale repack (package.rs:486-560),
  W13 fuse (package.rs:562-608).

``weight_shape`` is never read (the reference's tests require that it is not
loaded, weights/tests.rs:66-68,167-174).  An I32 word holds eight offset-binary
nibbles, element k at bits [4k, 4k+4), so on a little-endian host its bytes are
the byte-per-column-pair layout the repack kernels take.  Files are opened with
safetensors' own reader, which executes nothing from the file.
"""
from __future__ import annotations

import collections
import json
import os

import torch
from safetensors import safe_open

from . import ops

INDEX_FILE = "model.safetensors.index.json"
SINGLE_FILE = "model.safetensors"
LAYER_PREFIX = "language_model.model.layers."
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
COMPONENTS = ("weight_packed", "weight_scale")


def expert_tensor_name(layer: int, expert: int, projection: str, component: str) -> str:
    """Checkpoint name of one routed-expert tensor (manifest.rs:698-721)."""
    if projection not in PROJECTIONS or component not in COMPONENTS:
        raise ValueError(f"unknown expert tensor {projection}.{component}")
    return f"{LAYER_PREFIX}{layer}.mlp.experts.{expert}.{projection}.{component}"


class CheckpointIndex:
    """Tensor name -> shard file of a safetensors checkpoint directory."""

    def __init__(self, model_dir: str, weight_map: dict):
        self.model_dir = model_dir
        self.weight_map = weight_map

    @classmethod
    def from_model_dir(cls, model_dir: str) -> "CheckpointIndex":
        index_path = os.path.join(model_dir, INDEX_FILE)
        if os.path.exists(index_path):
            with open(index_path) as f:
                return cls.from_index_json(model_dir, json.load(f))
        single = os.path.join(model_dir, SINGLE_FILE)
        if os.path.exists(single):
            with safe_open(single, framework="pt") as f:
                return cls(model_dir, {name: SINGLE_FILE for name in f.keys()})
        raise FileNotFoundError(f"{model_dir} has neither {INDEX_FILE} nor {SINGLE_FILE}")

    @classmethod
    def from_index_json(cls, model_dir: str, index: dict) -> "CheckpointIndex":
        weight_map = index.get("weight_map") if isinstance(index, dict) else None
        if not isinstance(weight_map, dict):
            raise ValueError("safetensors index missing weight_map")
        for name, shard in weight_map.items():
            if not isinstance(shard, str):
                raise ValueError(f"weight_map entry {name} is not a shard string")
        return cls(model_dir, dict(weight_map))

    def shard_path(self, name: str) -> str:
        shard = self.weight_map.get(name)
        if shard is None:
            raise KeyError(f"checkpoint missing tensor {name}")
        return os.path.join(self.model_dir, shard)


def rank_expert_range(ep_rank: int, local_experts: int, global_experts: int) -> range:
    """Experts an EP rank owns: [rank * local, (rank + 1) * local)."""
    if local_experts <= 0 or ep_rank < 0 or (ep_rank + 1) * local_experts > global_experts:
        raise ValueError(f"EP rank {ep_rank} with {local_experts} local experts exceeds "
                         f"{global_experts} routed experts")
    return range(ep_rank * local_experts, (ep_rank + 1) * local_experts)


def projection_tensor_names(layer: int, experts: range, projection: str) -> list:
    """(packed, scale) names per expert, in expert order: everything one
    projection's load reads."""
    return [(expert_tensor_name(layer, e, projection, "weight_packed"),
             expert_tensor_name(layer, e, projection, "weight_scale")) for e in experts]


def read_projection(index: CheckpointIndex, layer: int, experts: range, projection: str,
                    out_dim: int, in_dim: int, group_size: int = 32):
    """Host tensors of one projection over `experts`, expert-major:
    (packed int32 [E, out, in/8], scale bf16 [E, out, in/group])."""
    if in_dim % 8 or in_dim % group_size:
        raise ValueError(f"in_dim {in_dim} must be a multiple of 8 and of {group_size}")
    names = projection_tensor_names(layer, experts, projection)
    E = len(names)
    packed = torch.empty((E, out_dim, in_dim // 8), dtype=torch.int32)
    scale = torch.empty((E, out_dim, in_dim // group_size), dtype=torch.bfloat16)
    want = {}
    for i, (pn, sn) in enumerate(names):
        want[pn] = (packed, i, torch.int32, (out_dim, in_dim // 8))
        want[sn] = (scale, i, torch.bfloat16, (out_dim, in_dim // group_size))
    by_shard = collections.defaultdict(list)
    for name in want:
        by_shard[index.shard_path(name)].append(name)
    for path, shard_names in by_shard.items():
        with safe_open(path, framework="pt") as f:
            present = set(f.keys())
            for name in shard_names:
                if name not in present:
                    raise KeyError(f"checkpoint tensor {name} is not in {os.path.basename(path)}")
                dst, i, dtype, shape = want[name]
                t = f.get_tensor(name)
                if t.dtype != dtype:
                    raise ValueError(f"{name}: dtype {t.dtype} does not match expected {dtype}")
                if tuple(t.shape) != shape:
                    raise ValueError(f"{name}: shape {tuple(t.shape)} does not match expected "
                                     f"{shape}")
                dst[i].copy_(t)
    return packed, scale


def load_routed_experts(model_dir: str, layer: int, ep_rank: int, *,
                        local_experts: int = ops.KIMI_K2_LOCAL_EXPERTS,
                        global_experts: int = ops.KIMI_K2_ROUTED_EXPERTS,
                        hidden: int = ops.KIMI_K2_HIDDEN,
                        inter: int = ops.KIMI_K2_EXPERT_INTERMEDIATE, device="cuda"):
    """(W13, W2) device packages of one MoE layer's local experts for one EP
    rank, ready for the grouped GEMM.  Kimi-K2 shapes (48 local of 384, hidden
    7168, intermediate 2048) go through the reference's repack entry points
    with its EP8 manifest; other shapes through the shape-general ones."""
    index = model_dir if isinstance(model_dir, CheckpointIndex) else \
        CheckpointIndex.from_model_dir(model_dir)
    experts = rank_expert_range(ep_rank, local_experts, global_experts)
    kimi = (local_experts, global_experts, hidden, inter) == (
        ops.KIMI_K2_LOCAL_EXPERTS, ops.KIMI_K2_ROUTED_EXPERTS, ops.KIMI_K2_HIDDEN,
        ops.KIMI_K2_EXPERT_INTERMEDIATE)
    roles = {"gate_proj": ops.KimiInt4ExpertRole.W1Gate, "up_proj": ops.KimiInt4ExpertRole.W3Up,
             "down_proj": ops.KimiInt4ExpertRole.W2Down}
    out = {}
    for proj in PROJECTIONS:
        out_dim, in_dim = (hidden, inter) if proj == "down_proj" else (inter, hidden)
        packed, scale = read_projection(index, layer, experts, proj, out_dim, in_dim)
        packed_d = packed.view(torch.uint8).reshape(-1).to(device)
        scale_d = scale.reshape(-1).to(device)
        if kimi:
            manifest = ops.KimiInt4WeightManifest.ep8(roles[proj], ep_rank,
                                                      ops.KimiInt4NibbleOrder.LowThenHigh)
            out[proj] = ops.kimi_marlin_int4_reorder(packed_d, scale_d, manifest)
        else:
            out[proj] = ops.marlin_int4_reorder(packed_d, scale_d, local_experts, in_dim, out_dim)
        del packed_d, scale_d
    return ops.marlin_int4_fuse_w13(out["gate_proj"], out["up_proj"]), out["down_proj"]
