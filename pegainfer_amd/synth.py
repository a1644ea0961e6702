"""Seeded synthetic inputs for the five benchmark configurations.

All generators are numpy (PCG64 seeded with 0x5EED0000 + config index and a
stream id), so tests and the CPU checker see identical bytes.  Checkpoint
tensors use the compressed-tensors layout the reference loads
(docs/models/kimi-k2/bringup-history.md:27-33 in the reference): packed
``[E, out, in/2]`` bytes, offset-binary nibbles (low nibble = even input
column, value = q + 8, q uniform in [-8, 7]) and bf16 scales ``[E, out, in/32]``
drawn as |N(0, 0.02)| / 7.
"""
from __future__ import annotations

import dataclasses

import numpy as np

SEED_BASE = 0x5EED0000


def rng(config_index: int, stream: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([SEED_BASE + config_index, stream]))


def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_bf16(g: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return bf16_bits(g.standard_normal(shape, dtype=np.float32) * np.float32(std))


def int4_checkpoint(g: np.random.Generator, experts: int, out_dim: int, in_dim: int,
                    group: int = 32, sigma: float = 0.02):
    """(packed uint8 [E, out, in/2], scales bf16 bits [E, out, in/group])."""
    packed = g.integers(0, 256, size=(experts, out_dim, in_dim // 2), dtype=np.uint8)
    z = np.abs(g.standard_normal((experts, out_dim, in_dim // group), dtype=np.float32))
    scales = bf16_bits(z * np.float32(sigma) / np.float32(7.0))
    return packed, scales


def fuse_checkpoint_w13(gate, up):
    """Logical fused W13 in checkpoint layout: rows [0, I) gate, [I, 2I) up."""
    (gp, gs), (up_, us) = gate, up
    return np.concatenate([gp, up_], axis=1), np.concatenate([gs, us], axis=1)


def zipf_local_topk(g: np.random.Generator, tokens: int, *, topk: int = 8, local_experts: int = 48,
                    global_experts: int = 384, s: float = 1.2, routes_target: int = 6600):
    """Kimi prefill routing with Zipf-skewed local hits: each token gets 1 or 2
    local slots (Bernoulli p = routes_target/tokens - 1) whose expert is drawn
    by Zipf(s) over ranks 1..local_experts (seeded rank -> expert permutation);
    the other slots get distinct non-local ids.  Weights are positive and sum
    to 1 per token."""
    p2 = min(max(routes_target / tokens - 1.0, 0.0), 1.0)
    ranks = np.arange(1, local_experts + 1, dtype=np.float64)
    prob = ranks ** (-s)
    prob /= prob.sum()
    perm = g.permutation(local_experts)
    idx = np.empty((tokens, topk), np.int32)
    nonlocal_pool = np.arange(local_experts, global_experts, dtype=np.int32)
    for t in range(tokens):
        n_local = 2 if g.random() < p2 else 1
        chosen = []
        while len(chosen) < n_local:
            e = int(perm[g.choice(local_experts, p=prob)])
            if e not in chosen:
                chosen.append(e)
        others = g.choice(nonlocal_pool, size=topk - n_local, replace=False)
        slots = np.array(chosen + list(others), np.int32)
        idx[t] = slots[g.permutation(topk)]
    w = g.random((tokens, topk), dtype=np.float32) + np.float32(0.1)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    index: int
    hidden: int
    inter: int
    experts: int
    topk: int
    tokens: int
    description: str


# BASELINE configurations (configs[0..4]).
C1 = Config("c1_dense_gemv_9728x2560", 1, 2560, 9728, 1, 1, 1,
            "dense W4A16 GEMV x[1,2560] . W[9728,2560]^T (Qwen3-4B MLP-up shape)")
C2 = Config("c2_kimi_expert_ffn", 2, 7168, 2048, 1, 1, 8,
            "one Kimi-K2 expert FFN, b in {1,4,8}: W13 [4096,7168] -> SwiGLU -> W2 [7168,2048]")
C3 = Config("c3_kimi_moe_decode_t64", 3, 7168, 2048, 48, 8, 64,
            "Kimi-K2 MoE layer, 48 of 384 experts, 64 decode tokens, sigmoid top-8")
C4 = Config("c4_dsv2lite_moe_prefill_t512", 4, 2048, 1408, 64, 6, 512,
            "DeepSeek-V2-Lite MoE layer, 64 experts top-6 softmax + 2 shared, 512 tokens")
C5 = Config("c5_kimi_prefill_t4096_zipf", 5, 7168, 2048, 48, 8, 4096,
            "Kimi-K2 local-expert prefill, 4096 tokens, Zipf(1.2) local routes")
CONFIGS = {c.name: c for c in (C1, C2, C3, C4, C5)}


def kimi_topk_margin(logits: np.ndarray, bias, topk: int = 8) -> np.ndarray:
    """Per token, the smallest gap between neighbours among the top topk + 1 of
    sigmoid(logit) + bias (fp64).  The Kimi router keeps its picks in selection
    order, so every neighbouring pair up to the first unpicked one decides the
    output; a gap well above a few fp32 ulps (1e-6) means exp implementations that
    differ by an ulp still pick the same indices in the same order."""
    s = 1.0 / (1.0 + np.exp(-np.asarray(logits, np.float64)))
    c = s + np.asarray(bias, np.float64)
    top = -np.sort(-c, axis=1)[:, :topk + 1]
    return (top[:, :-1] - top[:, 1:]).min(axis=1)


def dsv2_topk_margin(logits: np.ndarray, topk: int = 6) -> np.ndarray:
    """Per token, the gap between the topk-th and the next softmax probability
    (fp64).  The DeepSeek-V2-Lite router sorts its picks by expert id, so only this
    boundary decides the output."""
    l = np.asarray(logits, np.float64)
    p = np.exp(l - l.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    top = -np.sort(-p, axis=1)
    return top[:, topk - 1] - top[:, topk]
