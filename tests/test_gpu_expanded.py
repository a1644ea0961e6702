"""GPU parity of the expanded (expert-major) expert path, the DeepEP receive side of the
Kimi-K2 layer (pegainfer-kimi-k2/src/runner/moe_deepep.rs:332-385): routing metadata from
the post-epilogue prefix sum (K9) -> W13 over the expert-major buffer (top_k = 1,
experts.rs:1328-1360) -> SwiGLU reading the routed total on device (K3') -> W2 with one
bf16 top-k weight per row (experts.rs:1364-1401) -> residual join with the combined bf16
rows (kimi_residual_add_scaled_bf16).  The dispatch / combine collectives are out of scope
on one GPU: here every token has exactly one local route, so the combine is the row
permutation back to token order.  Each stage is checked against the oracle applied to the
GPU's own input to that stage (bit-exact where the stage is elementwise or integer work,
|gpu - ref| <= 1e-3 + 1e-2 |ref| for the GEMMs)."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_bf16_close, dev, host

pytestmark = pytest.mark.gpu


def test_deepep_expanded_sequence_kimi_shapes(oracle):
    from pegainfer_amd import layer, ops, synth
    E, H, I, T = 48, 7168, 2048, 64
    bs = align = 8  # DEEPEP_MARLIN_BLOCK (moe_deepep.rs:69)
    g = synth.rng(3, 21)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    w13 = layer.package_w13(gate, up)
    w2 = layer.package_projection(*down)
    rg = np.random.default_rng(5)
    expert_of_token = rg.integers(0, E, size=T)
    expert_of_token[:3] = 7  # one expert with several rows, some with none
    counts = np.bincount(expert_of_token, minlength=E)
    # expert-major layout with each segment starting at a multiple of the alignment
    starts = np.zeros(E, np.int64)
    psum = np.zeros(E + 1, np.int32)
    cur = 0
    for e in range(E):
        cur = -(-cur // align) * align
        starts[e] = cur
        cur += counts[e]
        psum[e] = cur
    psum[E] = -(-cur // align) * align
    capacity = int(psum[E]) + 5 * bs + 3  # room past the routed total, not a block multiple
    row_of_token = np.zeros(T, np.int64)
    fill = starts.copy()
    for t in range(T):
        e = expert_of_token[t]
        row_of_token[t] = fill[e]
        fill[e] += 1
    hidden = synth.normal_bf16(g, (T, H))
    recv_x = synth.normal_bf16(g, (capacity, H), std=50.0)  # pad rows hold garbage
    recv_x[row_of_token] = hidden
    recv_w = np.zeros(capacity, np.float32)
    recv_w[row_of_token] = rg.random(T).astype(np.float32) + 0.1

    route_ws = ops.KimiMarlinRouteWorkspace(capacity, bs)
    route_ws.sorted_token_ids.fill_(-9)
    route_ws.expert_ids.fill_(-9)
    routing = ops.kimi_deepep_build_marlin_routing_on_stream(route_ws, dev(psum), align, capacity)
    max_m_blocks = -(-capacity // bs)
    ref_r = oracle.deepep_build_routing(psum, E, align, bs, capacity, max_m_blocks)
    got_r = {"sorted_token_ids": host(route_ws.sorted_token_ids)[:capacity],
             "expert_ids": host(route_ws.expert_ids)[:max_m_blocks],
             "num_tokens_post_padded": host(route_ws.num_tokens_post_padded)}
    for k in got_r:
        assert np.array_equal(got_r[k], ref_r[k]), k
    assert got_r["num_tokens_post_padded"][0] == psum[E]
    # blocks past the routed total carry expert 0 and pad slots the capacity sentinel
    assert (got_r["expert_ids"][psum[E] // bs:] == 0).all()
    assert (got_r["sorted_token_ids"][psum[E]:] == capacity).all()

    gemm_ws = ops.KimiMarlinWna16Workspace(route_ws.max_m_blocks, max(2 * I, H), bs)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    w13_out = torch.zeros(capacity, 2 * I, **bf)
    act = torch.zeros(capacity, I, **bf)
    expert_out = torch.zeros(capacity, H, **bf)
    x_d, w_d = dev(recv_x), dev(recv_w)
    ops.kimi_marlin_wna16_expanded_w13_gemm(gemm_ws, routing, x_d, w13, w_d, w13_out)
    ops.kimi_marlin_w13_swiglu_expanded(w13_out, routing.num_tokens_post_padded, act, capacity, I)
    ops.kimi_marlin_wna16_expanded_w2_gemm(gemm_ws, routing, act, w2, w_d, expert_out)

    real = np.zeros(capacity, bool)
    real[row_of_token] = True
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    g13 = host(w13_out)
    ref13 = oracle.wna16_gemm(recv_x, w13p, w13s, ref_r, recv_w, moe_block_size=bs, top_k=1,
                              mul_topk_weights=False, size_m=capacity, size_n=2 * I, size_k=H,
                              threads=16)
    assert_bf16_close(g13[real], ref13[real], what="expanded W13")
    assert (g13[~real] == 0).all()  # pad rows are never written
    a = host(act)
    ntp = int(psum[E])
    assert np.array_equal(a[:ntp], oracle.swiglu(g13[:ntp], I))
    assert (a[ntp:] == 0).all()  # rows past the routed total are not touched
    eo = host(expert_out)
    ref2 = oracle.wna16_gemm(a, down[0], down[1], ref_r, recv_w, moe_block_size=bs, top_k=1,
                             mul_topk_weights=True, size_m=capacity, size_n=H, size_k=I,
                             threads=16)
    assert_bf16_close(eo[real], ref2[real], what="expanded W2")
    assert (eo[~real] == 0).all()

    # combine (one local route per token: a row permutation) and the residual join
    combined = eo[row_of_token]
    projected = synth.normal_bf16(g, (T, H), std=0.1)
    out = torch.zeros(T, H, **bf)
    ops.kimi_residual_add_scaled_bf16(dev(hidden), dev(projected), dev(combined),
                                      ops.KIMI_K2_ROUTER_SCALE, out)
    assert np.array_equal(host(out), oracle.residual_add_scaled_bf16(
        hidden, projected, combined, ops.KIMI_K2_ROUTER_SCALE))
    # end to end against the oracle's own chain (two GEMM tolerances composed)
    e2e = oracle.wna16_gemm(oracle.swiglu(ref13, I), down[0], down[1], ref_r, recv_w,
                            moe_block_size=bs, top_k=1, mul_topk_weights=True, size_m=capacity,
                            size_n=H, size_k=I, threads=16)
    assert_bf16_close(eo[real], e2e[real], rtol=2e-2, atol=2e-3, what="expanded end to end")
