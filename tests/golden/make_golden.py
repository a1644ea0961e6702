"""Writes the golden fixtures in this directory from the reference's own
known-answer tests (pure host code in the reference; no reference code is run).

Each fixture restates the *expected-value builder* of one reference test --
a formulation independent of the kernel it checks -- and stores inputs and
expected outputs as data:

* ``align_kat.npz``   -- pegainfer-kernels/src/ops/kimi_k2/experts.rs:1643-1728
  (56-entry topk_idx, global_start 96, block 8; expected = per local expert its
  route offsets ascending, padded with sentinel 56; expert_ids per block).
* ``scale_kat.npz``   -- experts.rs:1730-1796 (s(e,r,g)=bf16(e*0.25+r*0.01+g*0.125),
  in=out=64, 48 experts; expected via the source_flat formula of the test).
* ``weight_kat.npz``  -- experts.rs:1798-1902 (nibble (3e+5r+7c)&15, in=out=64,
  48 experts; expected via the test's sh_stage/warp/thread staging loop).
* ``misc_kat.npz``    -- experts.rs:1606-1628 (nibble decode, exhaustive),
  experts.rs:1630-1641 (capacity: 7 tokens, block 8 -> 49 m-blocks),
  pegainfer-deepseek-v2-lite/src/host_ops.rs:536-554 (top-6 sorted by id).

Run: ``python tests/golden/make_golden.py`` (deterministic; no randomness).
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LOCAL_EXPERTS = 48
TOPK = 8


def _bf16_bits(x_f32: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x_f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def align_kat():
    # experts.rs:1653-1657
    topk_host = [
        96, 97, 12, 143, 144, 98, 380, 99, 97, 96, 100, 101, 102, 103, 104, 105, 106, 107, 108,
        109, 110, 111, 112, 113, 96, 96, 96, 96, 96, 96, 96, 96, 120, 121, 122, 123, 124, 125,
        126, 127, 143, 143, 143, 143, 143, 143, 143, 143, 0, 383, 95, 144, 145, 146, 147, 148,
    ]
    active_tokens, block_size, global_start = 7, 8, 96
    route_elems = active_tokens * TOPK
    assert len(topk_host) == route_elems
    sentinel = route_elems
    expected_sorted, expected_expert_ids = [], []
    # experts.rs:1689-1711: builder over local experts
    for local_expert in range(LOCAL_EXPERTS):
        global_expert = global_start + local_expert
        routes = [off for off, ex in enumerate(topk_host) if ex == global_expert]
        if not routes:
            continue
        padded = -(-len(routes) // block_size) * block_size
        expected_expert_ids += [local_expert] * (padded // block_size)
        routes += [sentinel] * (padded - len(routes))
        expected_sorted += routes
    np.savez_compressed(
        os.path.join(HERE, "align_kat.npz"),
        topk_idx=np.array(topk_host, np.int32),
        active_tokens=np.int32(active_tokens), block_size=np.int32(block_size),
        global_start=np.int32(global_start), sentinel=np.int32(sentinel),
        expected_sorted=np.array(expected_sorted, np.int32),
        expected_expert_ids=np.array(expected_expert_ids, np.int32),
    )


def scale_kat():
    in_dim = out_dim = 64
    group_size = 32
    scale_k = in_dim // group_size
    epe = out_dim * scale_k
    e = np.arange(LOCAL_EXPERTS, dtype=np.float32)[:, None, None]
    r = np.arange(out_dim, dtype=np.float32)[None, :, None]
    g = np.arange(scale_k, dtype=np.float32)[None, None, :]
    # f32 arithmetic as in experts.rs:1744-1746 (no contraction)
    val = (e * np.float32(0.25)).astype(np.float32) + (r * np.float32(0.01)).astype(np.float32)
    val = val.astype(np.float32) + (g * np.float32(0.125)).astype(np.float32)
    checkpoint = _bf16_bits(val.astype(np.float32)).reshape(-1)
    expected = np.zeros_like(checkpoint)
    # experts.rs:1780-1794 (checked there for experts 0, 7, 47; the same map
    # holds for every expert)
    for expert in range(LOCAL_EXPERTS):
        for flat in range(epe):
            o = flat % 64
            source_flat = (flat // 64) * 64 + (o // 8 + 8 * (o % 8))
            group = source_flat // out_dim
            row = source_flat - group * out_dim
            expected[expert * epe + flat] = checkpoint[expert * epe + row * scale_k + group]
    np.savez_compressed(os.path.join(HERE, "scale_kat.npz"), in_dim=np.int32(in_dim),
                        out_dim=np.int32(out_dim), checkpoint=checkpoint, expected=expected)


def weight_kat():
    in_dim = out_dim = 64
    pack_factor, tile_k, tile_n = 8, 16, 64
    k_packed_cols = in_dim // pack_factor
    k_tiles, n_tiles = in_dim // tile_k, out_dim // tile_n
    wpe = out_dim * k_packed_cols

    def nibble(expert, row, col):
        return (expert * 3 + row * 5 + col * 7) & 0x0F

    checkpoint = np.zeros(LOCAL_EXPERTS * wpe, np.uint32)
    for expert in range(LOCAL_EXPERTS):
        for row in range(out_dim):
            for k_word in range(k_packed_cols):
                word = 0
                for pos in range(pack_factor):
                    word |= nibble(expert, row, k_word * pack_factor + pos) << (pos * 4)
                checkpoint[expert * wpe + row * k_packed_cols + k_word] = word
    expected = np.zeros_like(checkpoint)
    tc_offsets = [0, 1, 8, 9]
    pack_idx = [0, 2, 4, 6, 1, 3, 5, 7]
    # experts.rs:1823-1863 staging loop
    for expert in range(LOCAL_EXPERTS):
        cb, mb = expert * wpe, expert * wpe
        for k_tile in range(k_tiles):
            for n_tile in range(n_tiles):
                sh = [0] * (tile_n * (tile_k // pack_factor))
                for k_id in range(tile_k // pack_factor):
                    for n in range(tile_n):
                        sh[k_id * tile_n + n] = int(checkpoint[
                            cb + (n_tile * tile_n + n) * k_packed_cols
                            + k_tile * (tile_k // pack_factor) + k_id])
                for warp_id in range(4):
                    for th_id in range(32):
                        tc_col = th_id // 4
                        tc_row = (th_id % 4) * 2
                        cur_n = warp_id * 16 + tc_col
                        b1 = [sh[cur_n], sh[cur_n + tile_n]]
                        b2 = [sh[cur_n + 8], sh[cur_n + 8 + tile_n]]
                        vals = [0] * 8
                        for i in range(4):
                            cur_elem = tc_row + tc_offsets[i]
                            ci, cp = cur_elem // pack_factor, cur_elem % pack_factor
                            vals[i] = (b1[ci] >> (cp * 4)) & 0x0F
                            vals[4 + i] = (b2[ci] >> (cp * 4)) & 0x0F
                        packed = 0
                        for i in range(8):
                            packed |= vals[pack_idx[i]] << (i * 4)
                        tile_size = tile_k * tile_n // pack_factor
                        out_offset = (k_tile * n_tiles + n_tile) * tile_size
                        expected[mb + out_offset + th_id * 4 + warp_id] = packed
    np.savez_compressed(os.path.join(HERE, "weight_kat.npz"), in_dim=np.int32(in_dim),
                        out_dim=np.int32(out_dim), checkpoint=checkpoint, expected=expected)


def misc_kat():
    # experts.rs:1606-1628: byte = even | odd << 4, signed = nibble - 8
    bytes_ = np.arange(256, dtype=np.uint8)
    dec_even = (bytes_ & 0x0F).astype(np.int8) - 8
    dec_odd = ((bytes_ >> 4) & 0x0F).astype(np.int8) - 8
    # host_ops.rs:536-554: logits -10 except six, expected experts by id
    logits = np.full(64, -10.0, np.float32)
    for ex, lg in [(20, 6.0), (7, 5.0), (10, 4.0), (41, 3.0), (54, 2.0), (58, 1.0)]:
        logits[ex] = lg
    np.savez_compressed(
        os.path.join(HERE, "misc_kat.npz"),
        nibble_bytes=bytes_, nibble_even=dec_even, nibble_odd=dec_odd,
        capacity_tokens=np.int32(7), capacity_block=np.int32(8),
        capacity_expected_blocks=np.int32(49),
        capacity_expected_padded=np.int32(7 * TOPK + LOCAL_EXPERTS * 7),
        dsv2_logits=logits, dsv2_expected=np.array([7, 10, 20, 41, 54, 58], np.int32),
    )


if __name__ == "__main__":
    align_kat()
    scale_kat()
    weight_kat()
    misc_kat()
    print("golden fixtures written to", HERE)
