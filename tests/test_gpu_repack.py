"""GPU parity: load-time repacks (K5 weights, K6 scales, K7 W13 fuse) are
bit-exact with the reference's known-answer vectors and the oracle."""
import numpy as np
import pytest
import torch

from conftest import load_golden
from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def test_weight_repack_reference_kat():
    g = load_golden("weight_kat.npz")
    # the KAT uses in = out = 64, below the Kimi manifest shapes: call the C entry directly
    src = dev(g["checkpoint"].view(np.uint8))
    out = torch.full((g["checkpoint"].size * 4,), 0xAB, dtype=torch.uint8, device="cuda")
    from pegainfer_amd import _lib
    _lib.call("kimi_marlin_int4_reorder_weight_cuda", src.data_ptr(), out.data_ptr(), 64, 64, 48,
              32, torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host(out).view(np.uint32), g["expected"])


def test_scale_repack_reference_kat():
    from pegainfer_amd import _lib
    g = load_golden("scale_kat.npz")
    src = dev(g["checkpoint"])
    out = torch.zeros(g["checkpoint"].size, dtype=torch.bfloat16, device="cuda")
    _lib.call("kimi_marlin_int4_reorder_scale_cuda", src.data_ptr(), out.data_ptr(), 64, 64, 48,
              32, torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(host(out), g["expected"])


@pytest.mark.parametrize("E,K,N", [(1, 2560, 9728), (2, 7168, 256), (3, 2048, 7168 // 4)])
def test_repack_random_vs_oracle(oracle, E, K, N):
    from pegainfer_amd import ops
    g = np.random.default_rng(E * 7 + K)
    packed = g.integers(0, 256, size=(E, N, K // 2), dtype=np.uint8)
    scales = g.integers(0, 2 ** 16, size=(E, N, K // 32)).astype(np.uint16)
    w = ops.marlin_int4_reorder(dev(packed.reshape(-1)), dev(scales.reshape(-1)), E, K, N)
    ref_w = oracle.marlin_reorder_weight(packed.reshape(-1).view(np.uint32), K, N, E)
    ref_s = oracle.marlin_reorder_scale(scales.reshape(-1), K, N, E)
    assert np.array_equal(host(w.weight_packed_uint4b8).view(np.uint32), ref_w)
    assert np.array_equal(host(w.weight_scale_permuted), ref_s)


def test_fuse_w13_vs_oracle(oracle):
    from pegainfer_amd import ops
    g = np.random.default_rng(4)
    E, K, I = 48, 256, 128
    gp = g.integers(0, 256, size=(E, I, K // 2), dtype=np.uint8)
    up = g.integers(0, 256, size=(E, I, K // 2), dtype=np.uint8)
    gs = g.integers(0, 2 ** 16, size=(E, I, K // 32)).astype(np.uint16)
    us = g.integers(0, 2 ** 16, size=(E, I, K // 32)).astype(np.uint16)
    gw = ops.marlin_int4_reorder(dev(gp.reshape(-1)), dev(gs.reshape(-1)), E, K, I)
    uw = ops.marlin_int4_reorder(dev(up.reshape(-1)), dev(us.reshape(-1)), E, K, I)
    fused = ops.marlin_int4_fuse_w13(gw, uw)
    rgw = oracle.marlin_reorder_weight(gp.reshape(-1).view(np.uint32), K, I, E)
    ruw = oracle.marlin_reorder_weight(up.reshape(-1).view(np.uint32), K, I, E)
    rgs = oracle.marlin_reorder_scale(gs.reshape(-1), K, I, E)
    rus = oracle.marlin_reorder_scale(us.reshape(-1), K, I, E)
    ref_w, ref_s = oracle.marlin_fuse_w13(rgw, ruw, rgs, rus, K, I, E)
    assert np.array_equal(host(fused.weight_packed_uint4b8).view(np.uint32), ref_w)
    assert np.array_equal(host(fused.weight_scale_permuted), ref_s)
    # fusing per k-tile row equals repacking the concatenated [2I, K] checkpoint
    # (gate rows first), because the n-tiles of a k-tile row are contiguous.
    cat_p = np.concatenate([gp, up], axis=1)
    cat_s = np.concatenate([gs, us], axis=1)
    direct = oracle.marlin_reorder_weight(cat_p.reshape(-1).view(np.uint32), K, 2 * I, E)
    assert np.array_equal(direct, ref_w)
    direct_s = oracle.marlin_reorder_scale(cat_s.reshape(-1), K, 2 * I, E)
    assert np.array_equal(direct_s, ref_s)


def test_checkpoint_loader_gives_the_packed_layout(tmp_path):
    """checkpoint.load_routed_experts (safetensors shards -> W13/W2 device packages)
    equals packing the same experts' arrays directly, bit for bit."""
    from ckpt_helpers import write_checkpoint
    from pegainfer_amd import checkpoint, layer
    truth = write_checkpoint(str(tmp_path), experts=8, inter=128, hidden=256)
    w13, w2 = checkpoint.load_routed_experts(str(tmp_path), 3, 1, local_experts=4,
                                             global_experts=8, hidden=256, inter=128)
    stack = lambda proj: tuple(np.stack([truth[(e, proj)][i] for e in range(4, 8)])  # noqa: E731
                               for i in (0, 1))
    ref13 = layer.package_w13(stack("gate_proj"), stack("up_proj"))
    ref2 = layer.package_projection(*stack("down_proj"))
    for got, ref in ((w13, ref13), (w2, ref2)):
        assert (got.local_experts, got.in_dim, got.out_dim) == (ref.local_experts, ref.in_dim,
                                                                ref.out_dim)
        assert torch.equal(got.weight_packed_uint4b8, ref.weight_packed_uint4b8)
        assert torch.equal(got.weight_scale_permuted.view(torch.int16),
                           ref.weight_scale_permuted.view(torch.int16))
