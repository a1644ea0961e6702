"""GPU parity of whole expert-path configurations at BASELINE sizes (C1-C5).

Each layer is checked stage by stage -- every GPU stage against the oracle
applied to the GPU's own input to that stage, so errors cannot hide behind
compounding -- and end to end against the oracle's composite, all within
|gpu - ref| <= 1e-3 + 1e-2 |ref| (indices and permutations bit-exact).  The
4096-token prefill (C5) is checked on a sample of m-blocks (all rows of the
largest expert's first and last blocks plus random blocks) and through
size-independent properties on the rest.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_bf16_close, assert_f32_close, dev, host

pytestmark = pytest.mark.gpu


def _routing_host(r):
    return {"sorted_token_ids": host(r.sorted_token_ids), "expert_ids": host(r.expert_ids),
            "num_tokens_post_padded": host(r.num_tokens_post_padded)}


def _kimi_weights(cfg_index, E, H, I):
    from pegainfer_amd import synth
    g = synth.rng(cfg_index, 1)
    gate = synth.int4_checkpoint(g, E, I, H)
    up = synth.int4_checkpoint(g, E, I, H)
    down = synth.int4_checkpoint(g, E, H, I)
    return gate, up, down


def _routed_layer(gate, up, down, *, tokens, topk, block_size, global_start=0):
    from pegainfer_amd import layer
    w13 = layer.package_w13(gate, up)
    w2 = layer.package_projection(*down)
    return layer.RoutedExperts(w13, w2, max_tokens=tokens, topk=topk, block_size=block_size,
                               global_start=global_start)


def _unfused_w13(routed, hidden_dev, topk_w_dev, T):
    """The W13 GEMM alone (bf16 output) with the layer's routing, into a zeroed
    buffer.  The layer fuses SwiGLU into W13, so its activations must be SwiGLU of
    exactly these bits."""
    from pegainfer_amd import ops
    out = torch.zeros(T * routed.topk, 2 * routed.I, dtype=torch.bfloat16, device="cuda")
    ops.wna16_gemm(routed.gemm_ws, routed.routing, hidden_dev, routed.w13, topk_w_dev, out,
                   top_k=routed.topk, mul_topk_weights=False, size_m=T)
    return host(out)


def test_c1_dense_gemv(oracle):
    from pegainfer_amd import layer, synth
    g = synth.rng(1, 1)
    packed, scales = synth.int4_checkpoint(g, 1, 9728, 2560)
    x = synth.normal_bf16(synth.rng(1, 2), (1, 2560))
    dense = layer.DenseW4A16(layer.package_projection(packed, scales), max_rows=1)
    y = torch.zeros(1, 9728, dtype=torch.bfloat16, device="cuda")
    dense.forward(dev(x), y)
    routing = _routing_host(dense.routing)
    ref = oracle.wna16_gemm(x, packed, scales, routing, np.ones(1, np.float32), moe_block_size=8,
                            top_k=1, mul_topk_weights=False, size_m=1, size_n=9728, size_k=2560)
    assert_bf16_close(host(y), ref, what="C1")


@pytest.mark.parametrize("b", [1, 4, 8])
def test_c2_expert_ffn(oracle, b):
    from pegainfer_amd import layer, synth
    gate, up, down = _kimi_weights(2, 1, 7168, 2048)
    ffn = layer.ExpertFFN(layer.package_w13(gate, up), layer.package_projection(*down), max_rows=8)
    x = synth.normal_bf16(synth.rng(2, 2), (b, 7168))
    y = torch.zeros(b, 7168, dtype=torch.bfloat16, device="cuda")
    ffn.forward(dev(x), y, fused=False)  # the reference's call sequence, stage by stage
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    r_up = _routing_host(ffn.up.routing)
    h13 = host(ffn.h13[:b])
    ref13 = oracle.wna16_gemm(x, w13p, w13s, r_up, np.ones(b, np.float32), moe_block_size=8,
                              top_k=1, mul_topk_weights=False, size_m=b, size_n=4096, size_k=7168,
                              threads=8)
    assert_bf16_close(h13, ref13, what="C2 W13")
    act = host(ffn.act[:b])
    assert np.array_equal(act, oracle.swiglu(h13, 2048))
    r_dn = _routing_host(ffn.down.routing)
    ref2 = oracle.wna16_gemm(act, down[0], down[1], r_dn, np.ones(b, np.float32), moe_block_size=8,
                             top_k=1, mul_topk_weights=False, size_m=b, size_n=7168, size_k=2048,
                             threads=8)
    assert_bf16_close(host(y), ref2, what="C2 W2")
    # end to end against the oracle's own chain
    e2e = oracle.wna16_gemm(oracle.swiglu(ref13, 2048), down[0], down[1], r_dn,
                            np.ones(b, np.float32), moe_block_size=8, top_k=1,
                            mul_topk_weights=False, size_m=b, size_n=7168, size_k=2048, threads=8)
    assert_bf16_close(host(y), e2e, rtol=2e-2, atol=2e-3, what="C2 end to end")
    # the fused W13 + SwiGLU path (split K, partials summed by the SwiGLU kernel)
    y_fused = torch.zeros_like(y)
    ffn.forward(dev(x), y_fused, fused=True)
    assert_bf16_close(host(ffn.act[:b]), oracle.swiglu(ref13, 2048), rtol=2e-2, atol=2e-3,
                      what="C2 fused SwiGLU")
    assert_bf16_close(host(y_fused), e2e, rtol=2e-2, atol=2e-3, what="C2 fused end to end")


def test_c3_kimi_decode_layer(oracle):
    from pegainfer_amd import ops, synth
    E, H, I, T = 48, 7168, 2048, 64
    gate, up, down = _kimi_weights(3, E, H, I)
    hidden = synth.normal_bf16(synth.rng(3, 2), (T, H))
    logits = synth.rng(3, 3).standard_normal((T, 384), dtype=np.float32)
    bias = np.zeros(384, np.float32)
    # neighbouring score + bias values among each token's top 9 differ by far more than
    # an ulp: the picks and their order do not depend on the exp implementation
    assert synth.kimi_topk_margin(logits, bias).min() > 1e-6
    bs = ops.kimi_marlin_block_size(T)
    assert bs == 16
    moe = _routed_layer(gate, up, down, tokens=T, topk=8, block_size=bs)
    w = torch.zeros(T, 8, dtype=torch.float32, device="cuda")
    idx = torch.zeros(T, 8, dtype=torch.int32, device="cuda")
    ops.kimi_router_select(dev(logits), dev(bias), w, idx, T)
    ref_idx, ref_w = oracle.kimi_router(logits, bias, 8, 1.0)
    assert np.array_equal(host(idx), ref_idx) and np.array_equal(host(w), ref_w)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    # a first call with other routes leaves stale rows behind: the default flow
    # skips the zero-fills, so only rows of local routes may be compared below
    hidden_d = dev(hidden)
    moe.forward(hidden_d, ((idx + 11) % 384).contiguous(), w, out)
    moe.forward(hidden_d, idx, w, out)
    local = (ref_idx.reshape(-1) < E)

    routing = _routing_host(moe.routing)
    ref_r = oracle.align_block_size(ref_idx.reshape(-1), 0, E, bs)
    assert np.array_equal(routing["sorted_token_ids"], ref_r["sorted_token_ids"])
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    g13 = _unfused_w13(moe, hidden_d, w, T)  # the layer fuses SwiGLU into W13
    ref13 = oracle.wna16_gemm(hidden, w13p, w13s, routing, ref_w, moe_block_size=bs, top_k=8,
                              mul_topk_weights=False, size_m=T, size_n=2 * I, size_k=H, threads=16)
    assert_bf16_close(g13[local], ref13[local], what="C3 W13")
    act = host(moe.act[:T * 8])
    assert np.array_equal(act[local], oracle.swiglu(g13, I)[local])
    act[~local] = 0
    ro = host(moe.route_out[:T * 8])
    ref2 = oracle.wna16_gemm(act, down[0], down[1], routing, ref_w, moe_block_size=bs, top_k=1,
                             mul_topk_weights=True, size_m=T * 8, size_n=H, size_k=I, threads=16)
    assert_bf16_close(ro[local], ref2[local], what="C3 W2")
    ro[~local] = 0
    got = host(out)
    assert np.array_equal(got, oracle.sum_topk_rows(ro, T, 8, H))
    # the reference's call sequence (zero-fills, W13 then SwiGLU, full combine) gives the
    # same bits
    out_ref_flow = torch.zeros_like(out)
    moe.forward(dev(hidden), idx, w, out_ref_flow, reference_flow=True)
    assert np.array_equal(host(out_ref_flow).view(np.uint32), got.view(np.uint32))
    ref_out, _ = oracle.kimi_moe_layer(hidden, w13p, w13s, down[0], down[1], ref_idx.reshape(-1),
                                       ref_w, global_start=0, local_experts=E, block_size=bs,
                                       hidden=H, inter=I, threads=16)
    assert_f32_close(got, ref_out, rtol=2e-2, atol=2e-3, what="C3 end to end")


def test_c4_dsv2_layer(oracle):
    from pegainfer_amd import layer, ops, synth
    E, H, I, T, topk = 64, 2048, 1408, 512, 6
    g = synth.rng(4, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    sg, su, sd = (synth.int4_checkpoint(g, 1, 2 * I, H), synth.int4_checkpoint(g, 1, 2 * I, H),
                  synth.int4_checkpoint(g, 1, H, 2 * I))
    hidden = synth.normal_bf16(synth.rng(4, 2), (T, H))
    logits = synth.rng(4, 3).standard_normal((T, E), dtype=np.float32)
    # every token's 6th/7th probability gap is far above an ulp: the selected set does
    # not depend on the exp implementation
    assert synth.dsv2_topk_margin(logits, topk).min() > 1e-6
    bs = ops.kimi_marlin_block_size(T, topk=topk, local_experts=E)
    routed = _routed_layer(gate, up, down, tokens=T, topk=topk, block_size=bs)
    shared = layer.ExpertFFN(layer.package_w13(sg, su), layer.package_projection(*sd), max_rows=T)
    moe = layer.Dsv2MoeLayer(routed, shared)
    out = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
    hidden_d = dev(hidden)
    moe.forward(hidden_d, dev(logits), out)

    ref_idx, ref_w = oracle.dsv2_router(logits, topk)
    assert np.array_equal(host(moe.topk_idx), ref_idx) and np.array_equal(host(moe.topk_w), ref_w)
    routing = _routing_host(routed.routing)
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    g13 = _unfused_w13(routed, hidden_d, moe.topk_w, T)
    ref13 = oracle.wna16_gemm(hidden, w13p, w13s, routing, ref_w, moe_block_size=bs, top_k=topk,
                              mul_topk_weights=False, size_m=T, size_n=2 * I, size_k=H, threads=16)
    assert_bf16_close(g13, ref13, what="C4 W13")
    act = host(routed.act[:T * topk])
    assert np.array_equal(act, oracle.swiglu(g13, I))
    ro = host(routed.route_out[:T * topk])
    ref2 = oracle.wna16_gemm(act, down[0], down[1], routing, ref_w, moe_block_size=bs, top_k=1,
                             mul_topk_weights=False, size_m=T * topk, size_n=H, size_k=I,
                             threads=16)
    assert_bf16_close(ro, ref2, what="C4 W2")
    routed_f32 = oracle.weighted_topk_sum(ro, ref_w, T, topk, H)
    sh = host(moe.shared_out)
    # the combine and the join as the reference rounds them, bf16(f(bf16(routed)) + f(shared)),
    # here in one launch
    assert np.array_equal(host(out), oracle.dsv2_join(routed_f32, sh))
    # the shared expert: one INT4 expert over all tokens (W13 + SwiGLU fused, then W2)
    sI = 2 * I
    sbs = shared.up.block_size
    h13 = torch.zeros(T, 2 * sI, dtype=torch.bfloat16, device="cuda")
    shared.up.forward(hidden_d, h13)  # the W13 GEMM alone, same routing
    g13s = host(h13)
    r_up = _routing_host(shared.up.routing)
    ref13s = oracle.wna16_gemm(hidden, np.concatenate([sg[0], su[0]], axis=1),
                               np.concatenate([sg[1], su[1]], axis=1), r_up,
                               np.ones(T, np.float32), moe_block_size=sbs, top_k=1,
                               mul_topk_weights=False, size_m=T, size_n=2 * sI, size_k=H,
                               threads=16)
    assert_bf16_close(g13s, ref13s, what="C4 shared W13")
    act_s = host(shared.act[:T])
    assert np.array_equal(act_s, oracle.swiglu(g13s, sI))
    r_dn = _routing_host(shared.down.routing)
    ref2s = oracle.wna16_gemm(act_s, sd[0], sd[1], r_dn, np.ones(T, np.float32),
                              moe_block_size=sbs, top_k=1, mul_topk_weights=False, size_m=T,
                              size_n=H, size_k=sI, threads=16)
    assert_bf16_close(sh, ref2s, what="C4 shared W2")
    # prefill block sizes: each shared-expert GEMM runs in the routed GEMM's launch,
    # with the bits of the serial order
    assert moe.pair
    serial = layer.Dsv2MoeLayer(routed, shared, overlap_shared=False)
    out_serial = torch.zeros_like(out)
    serial.forward(hidden_d, dev(logits), out_serial)
    assert np.array_equal(host(out_serial), host(out))
    # the serial flow keeps the combine and the join apart: its fp32 rows are the oracle's
    assert np.array_equal(host(serial.routed_f32), routed_f32)


def test_c5_kimi_prefill_sampled(oracle):
    from pegainfer_amd import ops, synth
    E, H, I, T = 48, 7168, 2048, 4096
    gate, up, down = _kimi_weights(5, E, H, I)
    hidden = synth.normal_bf16(synth.rng(5, 2), (T, H))
    idx, w = synth.zipf_local_topk(synth.rng(5, 3), T)
    bs = ops.kimi_marlin_block_size(T)
    moe = _routed_layer(gate, up, down, tokens=T, topk=8, block_size=bs)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    hidden_d, w_d = dev(hidden), dev(w)
    moe.forward(hidden_d, dev(idx), w_d, out)
    routing = _routing_host(moe.routing)
    ref_r = oracle.align_block_size(idx.reshape(-1), 0, E, bs)
    for k in ("sorted_token_ids", "expert_ids", "num_tokens_post_padded"):
        assert np.array_equal(routing[k], ref_r[k]), k

    nblocks = int(routing["num_tokens_post_padded"][0]) // bs
    eids = routing["expert_ids"][:nblocks]
    big = np.bincount(eids).argmax()
    big_blocks = np.flatnonzero(eids == big)
    g = np.random.default_rng(0)
    sample = sorted(set([big_blocks[0], big_blocks[-1]] + list(g.choice(nblocks, 6, replace=False))))
    masked = dict(routing)
    masked["expert_ids"] = np.where(np.isin(np.arange(routing["expert_ids"].size), sample),
                                    routing["expert_ids"], -1).astype(np.int32)
    rows = np.concatenate([routing["sorted_token_ids"][b * bs:(b + 1) * bs] for b in sample])
    rows = rows[rows < T * 8]
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    g13 = _unfused_w13(moe, hidden_d, w_d, T)
    ref13 = oracle.wna16_gemm(hidden, w13p, w13s, masked, w, moe_block_size=bs, top_k=8,
                              mul_topk_weights=False, size_m=T, size_n=2 * I, size_k=H, threads=16)
    assert_bf16_close(g13[rows], ref13[rows], what="C5 W13 sampled blocks")
    act = host(moe.act[:T * 8])
    assert np.array_equal(act[rows], oracle.swiglu(g13[rows], I))
    ro = host(moe.route_out[:T * 8])
    ref2 = oracle.wna16_gemm(act, down[0], down[1], masked, w, moe_block_size=bs, top_k=1,
                             mul_topk_weights=True, size_m=T * 8, size_n=H, size_k=I, threads=16)
    assert_bf16_close(ro[rows], ref2[rows], what="C5 W2 sampled blocks")
    # properties on every row: the GEMMs never write rows of non-local routes
    # (this layer's buffers start at zero); the combine is the exact fp32 sum of
    # the routed rows
    local = (idx.reshape(-1) < E)
    assert (ro[~local] == 0).all() and (g13[~local] == 0).all() and (act[~local] == 0).all()
    assert np.array_equal(act[local], oracle.swiglu(g13[local], I))
    assert (np.abs((ro[local].astype(np.uint32) << 16).view(np.float32)).sum(axis=1) > 0).all()
    assert np.array_equal(host(out), oracle.sum_topk_rows(ro, T, 8, H))


def _exact_int4(g, E, N, K):
    """Checkpoint tensors whose dequantised weights are q * 2^e, e in {-2, -1, 0}: with
    small-integer activations every product and partial sum of a K <= 7168 dot product
    is an exact fp32 number (magnitudes below 2^18 on a 2^-2 grid), so any summation
    order gives the same fp32 sum and a float32 BLAS product reproduces it exactly."""
    from oracle import oracle
    q = g.integers(-8, 8, size=(E, N, K), dtype=np.int8)
    exps = g.integers(-2, 1, size=(E, N, K // 32))
    scales_f = np.ldexp(np.float32(1.0), exps).astype(np.float32)
    u = (q + 8).astype(np.uint8)
    packed = (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)
    return (packed, oracle.f32_to_bf16(scales_f)), q, scales_f


def _exact_rows(a_f32, q_e, s_e):
    """fp32 [rows, N] = a . (q * s)^T, exact for the inputs of _exact_int4."""
    w = (q_e.astype(np.float32) * np.repeat(s_e, 32, axis=1)).astype(np.float32)
    return a_f32 @ w.T


def test_c5_every_block_exact_inputs(oracle):
    """C5's routing at full size (4096 tokens, 6565 Zipf routes, every m-block of all 48
    experts) with exact inputs: every routed row of W13 must equal the float32 product
    rounded to bf16 bit for bit, the fused SwiGLU must be SwiGLU of those bits, and every
    routed W2 row (exact activations fed in, bf16 top-k weight applied) likewise."""
    from pegainfer_amd import ops, synth
    E, H, I, T = 48, 7168, 2048, 4096
    g = np.random.default_rng(0x5EED0005)
    (gp, gs), qg, sg = _exact_int4(g, E, I, H)
    (upk, us), qu, su = _exact_int4(g, E, I, H)
    (dp, ds), qd, sd = _exact_int4(g, E, H, I)
    a = g.integers(-2, 3, size=(T, H)).astype(np.float32)
    idx, w = synth.zipf_local_topk(synth.rng(5, 3), T)
    bs = ops.kimi_marlin_block_size(T)
    moe = _routed_layer((gp, gs), (upk, us), (dp, ds), tokens=T, topk=8, block_size=bs)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    a_bits = oracle.f32_to_bf16(a)
    hidden_d, w_d, idx_d = dev(a_bits), dev(w), dev(idx)
    moe.forward(hidden_d, idx_d, w_d, out)
    g13 = _unfused_w13(moe, hidden_d, w_d, T)
    act = host(moe.act[:T * 8])
    flat = idx.reshape(-1)
    local = flat < E
    routing = _routing_host(moe.routing)
    nblocks = int(routing["num_tokens_post_padded"][0]) // bs
    assert nblocks > 100 and np.unique(routing["expert_ids"][:nblocks]).size == E
    qw13 = np.concatenate([qg, qu], axis=1)
    sw13 = np.concatenate([sg, su], axis=1)
    for e in range(E):
        rows = np.flatnonzero(flat == e)
        want = oracle.f32_to_bf16(_exact_rows(a[rows // 8], qw13[e], sw13[e]))
        assert np.array_equal(g13[rows], want), f"W13 expert {e}"
    assert np.array_equal(act[local], oracle.swiglu(g13[local], I))
    # W2 over every routed row, with exact activations
    act_x = np.zeros((T * 8, I), np.float32)
    act_x[local] = g.integers(-3, 4, size=(int(local.sum()), I))
    ro = torch.zeros(T * 8, H, dtype=torch.bfloat16, device="cuda")
    ops.wna16_gemm(moe.gemm_ws, moe.routing, dev(oracle.f32_to_bf16(act_x)), moe.w2, w_d, ro,
                   top_k=1, mul_topk_weights=True, size_m=T * 8)
    ro = host(ro)
    twb = oracle.bf16_to_f32(oracle.f32_to_bf16(w.reshape(-1)))
    for e in range(E):
        rows = np.flatnonzero(flat == e)
        acc = oracle.f32_to_bf16(_exact_rows(act_x[rows], qd[e], sd[e]))
        want = oracle.f32_to_bf16(oracle.bf16_to_f32(acc) * twb[rows][:, None])
        assert np.array_equal(ro[rows], want), f"W2 expert {e}"
    assert (ro[~local] == 0).all()


@pytest.mark.parametrize("E", [48, 8])
def test_routed_layer_edge_batches(oracle, E):
    """The routed-expert layer at the batch edges, each against the oracle's composite and
    against the reference's own call sequence (zero-fills, unfused SwiGLU, full combine), bit
    for bit at the prefill block sizes: one token; a batch with no local route at all (the output must be zero); a
    decode batch after a larger prefill-size one on the same buffers (stale rows of the
    earlier call must not leak); the prefill block sizes at a few tokens.  E = 48 runs the
    reference's kimi_* symbols, E = 8 the shape-general entries."""
    from pegainfer_amd import ops, synth
    H, I, topk = 512, 256, 8
    gate, up, down = _kimi_weights(7, E, H, I)
    w13p = np.concatenate([gate[0], up[0]], axis=1)
    w13s = np.concatenate([gate[1], up[1]], axis=1)
    g = np.random.default_rng(0xED6E)
    # (tokens, block size, local routes?, what); each block size sees a larger batch
    # before the smaller ones on the same layer buffers
    cases = [(1, ops.kimi_marlin_block_size(1, topk, E), True, "one token, policy block size"),
             (64, 16, True, "decode batch"), (1, 16, True, "one token after 64"),
             (5, 16, False, "no local route"), (200, 64, True, "prefill size"),
             (3, 64, True, "three tokens after 200, block 64"), (40, 32, True, "block 32"),
             (7, 32, True, "seven tokens after 40, block 32"), (9, 8, True, "block 8")]
    layers = {}
    for T, bs, any_local, what in cases:
        if bs not in layers:
            layers[bs] = _routed_layer(gate, up, down, tokens=256, topk=topk, block_size=bs)
        moe = layers[bs]
        if not any_local:
            idx = g.integers(E, 4 * E, size=(T, topk)).astype(np.int32)
        else:
            idx = np.stack([g.permutation(4 * E)[:topk] for _ in range(T)]).astype(np.int32)
        w = g.random((T, topk), dtype=np.float32)
        hidden = synth.normal_bf16(g, (T, H))
        out = torch.full((T, H), np.nan, dtype=torch.float32, device="cuda")
        moe.forward(dev(hidden), dev(idx), dev(w), out)
        got = host(out)
        ref_flow = torch.full((T, H), np.nan, dtype=torch.float32, device="cuda")
        moe.forward(dev(hidden), dev(idx), dev(w), ref_flow, reference_flow=True)
        if bs > 16:
            # one wave covers all of K in both W13 forms: the same fp32 sums
            assert np.array_equal(host(ref_flow).view(np.uint32), got.view(np.uint32)), what
        else:
            # these small decode grids split K one way in the fused W13 (across
            # workgroups, or 8 waves) and another in the plain GEMM (16 waves, or 2)
            assert_f32_close(got, host(ref_flow), rtol=2e-2, atol=2e-3, what=what)
        if not any_local:
            assert (got == 0).all(), what
            continue
        ref, _ = oracle.kimi_moe_layer(hidden, w13p, w13s, down[0], down[1], idx.reshape(-1), w,
                                       global_start=0, local_experts=E, block_size=bs, hidden=H,
                                       inter=I, topk=topk, threads=8)
        assert_f32_close(got, ref, rtol=2e-2, atol=2e-3, what=f"{what} (T={T}, bs={bs})")
