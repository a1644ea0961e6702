"""GPU parity on the deterministic synthetic inputs of the reference's own comparison tool
against vLLM's Marlin MoE GEMM (pegainfer-kernels/tools/kimi_k2/vllm_marlin_wna16_reference.py:
26-48 and 166-191), at Kimi-K2 shapes (48 local experts, hidden 7168, intermediate 2048, top-8):

* hidden[i] = ((i mod 23) - 11) / 32;
* route r of token t goes to expert (13 t + 5 r) mod 48 with weight (r + 1) / 36;
* the packed weights are written straight into the device (Marlin) layout from the tool's
  generator (i * 1103515245 + 12345 + (i // 97) * 17) & 0x7fffffff;
* the group scales are ((i mod 17) + 1) / 64 (W13) and ((i mod 19) + 1) / 64 (W2) in the
  [expert, k/32, n] order the tool builds, permuted by the library's scale repack (the
  permutation the tool gets from vLLM's marlin_moe_permute_scales).

The tool's outputs are not part of the reference, so the expected values come from the CPU
oracle fed the same weights unpacked to checkpoint order.  With these inputs every W13 product
is a multiple of 2^-11 and every partial sum stays below 2^13, so the W13 sums are exact in
fp32 in any order: W13, the fused SwiGLU and the top-k sum must match bit for bit.  W2 (whose
inputs are the SwiGLU outputs) is held to the fp32 summation error bound before its top-k
weight, and bit for bit after it given the unweighted bits.

T = 4, 64, 160, 250, 400 and 4096 take block sizes 8, 16, 32, 48, 64 and 64 (the decode
K-split path, the 16x16x32 decode kernel, and the prefill kernel at three block sizes up to
the full C5 token count, where every one of the 32768 routes is local).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu

E, H, I, TOPK = 48, 7168, 2048, 8


def _lcg_words(numel):
    """fill_qweight (vllm_marlin_wna16_reference.py:26-29) as uint32 words."""
    idx = np.arange(numel, dtype=np.int64)
    return ((idx * 1103515245 + 12345 + (idx // 97) * 17) & 0x7FFFFFFF).astype(np.uint32)


def _fill_bf16(oracle, numel, modulo, scale, offset):
    """fill_bf16 (vllm_marlin_wna16_reference.py:32-35): exact bf16 values here."""
    idx = np.arange(numel, dtype=np.int64)
    return oracle.f32_to_bf16(((idx % modulo).astype(np.float32) + np.float32(offset))
                              * np.float32(scale))


def _projection(oracle, in_dim, out_dim, modulo):
    """(device weight, checkpoint u8 [E, out, in/2], checkpoint scales [E, out, in/32])."""
    from pegainfer_amd import ops
    words = _lcg_words(E * (in_dim // 16) * (out_dim * 2))
    raw_scale = _fill_bf16(oracle, E * (in_dim // 32) * out_dim, modulo, 1.0 / 64.0, 1.0)
    ckpt_scale = np.ascontiguousarray(
        raw_scale.reshape(E, in_dim // 32, out_dim).transpose(0, 2, 1))
    ckpt_words = oracle.marlin_unpack_weight(words, in_dim, out_dim, E)
    ckpt_u8 = ckpt_words.view(np.uint8).reshape(E, out_dim, in_dim // 2)
    from pegainfer_amd import _lib
    src = dev(ckpt_scale)
    scale = torch.empty(ckpt_scale.size, dtype=torch.bfloat16, device="cuda")
    _lib.call("pega_marlin_int4_reorder_scale", src.data_ptr(), scale.data_ptr(), in_dim,
              out_dim, E, 32, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    packed = torch.from_numpy(words.view(np.uint8)).cuda()
    w = ops.MarlinInt4Weight(E, in_dim, out_dim, packed, scale)
    return w, ckpt_u8, ckpt_scale


@pytest.fixture(scope="module")
def kimi_weights(oracle):
    w13 = _projection(oracle, H, 2 * I, 17)
    w2 = _projection(oracle, I, H, 19)
    torch.cuda.synchronize()
    return w13, w2


@pytest.mark.parametrize("T", [4, 64, 160, 250, 400, 4096])
def test_reference_tool_inputs(oracle, kimi_weights, T):
    from pegainfer_amd import layer, ops
    (w13, q13, s13), (w2, q2, s2) = kimi_weights
    hidden = _fill_bf16(oracle, T * H, 23, 1.0 / 32.0, -11.0).reshape(T, H)
    t, r = np.meshgrid(np.arange(T), np.arange(TOPK), indexing="ij")
    idx = ((13 * t + 5 * r) % E).astype(np.int32)
    w = np.tile(np.arange(1, TOPK + 1, dtype=np.float32) / np.float32(36.0), (T, 1))
    bs = ops.kimi_marlin_block_size(T)
    moe = layer.RoutedExperts(w13, w2, max_tokens=T, topk=TOPK, block_size=bs)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    hidden_d, w_d = dev(hidden), dev(w)
    moe.forward(hidden_d, dev(idx), w_d, out)
    routing = {k: host(v) for k, v in (("sorted_token_ids", moe.routing.sorted_token_ids),
                                       ("expert_ids", moe.routing.expert_ids),
                                       ("num_tokens_post_padded",
                                        moe.routing.num_tokens_post_padded))}
    # W13 alone (bf16 output), then the fused W13 + SwiGLU the layer ran
    g13 = torch.zeros(T * TOPK, 2 * I, dtype=torch.bfloat16, device="cuda")
    ops.wna16_gemm(moe.gemm_ws, moe.routing, hidden_d, w13, w_d, g13, top_k=TOPK,
                   mul_topk_weights=False, size_m=T)
    ref13 = oracle.wna16_gemm(hidden, q13, s13, routing, w, moe_block_size=bs, top_k=TOPK,
                              mul_topk_weights=False, size_m=T, size_n=2 * I, size_k=H,
                              threads=16, fast=True)
    assert np.array_equal(host(g13), ref13), f"W13 T={T}"
    act = host(moe.act[:T * TOPK])
    assert np.array_equal(act, oracle.swiglu(ref13, I)), f"fused SwiGLU T={T}"
    # W2 without the top-k weight against the oracle, then the layer's weighted W2 exactly
    # as bf16(bf16(sum) * bf16(weight)) of those bits.  These inputs make W2 ill-conditioned:
    # the SwiGLU outputs reach ~1e7 and a row's 2048 products cancel to values near 1, so two
    # fp32 summation orders legitimately differ by far more than rel 1e-2 of the result.  The
    # bound is therefore the one any fp32 sum of n terms obeys, |sum - exact| <= g(n) S with
    # g(n) = n u / (1 - n u), u = 2^-24 and S the sum of the terms' magnitudes (both sides),
    # plus one bf16 ulp for the two final roundings; S comes from float64 products of the
    # same (exactly representable) dequantised weights.
    plain = torch.zeros(T * TOPK, H, dtype=torch.bfloat16, device="cuda")
    ops.wna16_gemm(moe.gemm_ws, moe.routing, dev(act), w2, w_d, plain, top_k=1,
                   mul_topk_weights=False, size_m=T * TOPK)
    plain = oracle.bf16_to_f32(host(plain)).astype(np.float64)
    ref2 = oracle.bf16_to_f32(oracle.wna16_gemm(
        act, q2, s2, routing, w, moe_block_size=bs, top_k=1, mul_topk_weights=False,
        size_m=T * TOPK, size_n=H, size_k=I, threads=16, fast=True)).astype(np.float64)
    act64 = np.abs(oracle.bf16_to_f32(act).astype(np.float64))
    flat = idx.reshape(-1)
    u = 2.0 ** -24
    gamma = I * u / (1 - I * u)
    for e in np.unique(flat):
        rows = np.flatnonzero(flat == e)
        nib = np.stack([q2[e] & 15, q2[e] >> 4], axis=-1).reshape(H, I).astype(np.float64) - 8
        wde = np.abs(nib * np.repeat(oracle.bf16_to_f32(s2[e]).astype(np.float64), 32, axis=1))
        bound_s = act64[rows] @ wde.T
        big = np.maximum(np.abs(plain[rows]), np.abs(ref2[rows]))
        ulp = np.ldexp(1.0, np.floor(np.log2(np.maximum(big, 2.0 ** -126))).astype(int) - 7)
        err = np.abs(plain[rows] - ref2[rows])
        assert (err <= 2 * gamma * bound_s + ulp).all(), f"W2 expert {e} T={T}"
    plain = oracle.f32_to_bf16(plain.astype(np.float32))
    ro = host(moe.route_out[:T * TOPK])
    wb = oracle.bf16_to_f32(oracle.f32_to_bf16(w.reshape(-1)))
    assert np.array_equal(ro, oracle.f32_to_bf16(oracle.bf16_to_f32(plain) * wb[:, None])), \
        f"W2 top-k weight T={T}"
    assert np.array_equal(host(out), oracle.sum_topk_rows(ro, T, TOPK, H)), f"combine T={T}"
