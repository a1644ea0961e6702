"""GPU parity: token -> expert permutation (K1), DeepEP routing metadata (K9)
and the router select stages, bit-exact against the oracle and the
reference's known-answer vector."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import load_golden
from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def _gpu_align(topk_idx, tokens, topk, global_start, E, bs, kimi=True):
    from pegainfer_amd import ops
    ws = ops.KimiMarlinRouteWorkspace(tokens, bs, topk=topk, local_experts=E)
    # poison the outputs so that untouched slots are visible
    for t in (ws.sorted_token_ids, ws.expert_ids, ws.expert_offsets, ws.expert_cursor):
        t.fill_(-7)
    routing = ops.moe_align_block_size(ws, dev(np.ascontiguousarray(topk_idx, np.int32).reshape(-1)),
                                       tokens, tokens, global_start)
    return ws, routing


def _check_against_oracle(oracle, ws, topk_idx, global_start, E, bs):
    ref = oracle.align_block_size(np.asarray(topk_idx, np.int32).reshape(-1), global_start, E, bs,
                                  ws.max_padded_tokens, ws.max_m_blocks)
    assert np.array_equal(host(ws.sorted_token_ids), ref["sorted_token_ids"])
    assert np.array_equal(host(ws.expert_ids), ref["expert_ids"])
    assert np.array_equal(host(ws.num_tokens_post_padded), ref["num_tokens_post_padded"])
    assert np.array_equal(host(ws.expert_offsets).view(np.uint32), ref["expert_offsets"])
    assert np.array_equal(host(ws.expert_cursor).view(np.uint32), ref["expert_cursor"])


def test_align_reference_kat():
    g = load_golden("align_kat.npz")
    ws, routing = _gpu_align(g["topk_idx"], int(g["active_tokens"]), 8, int(g["global_start"]),
                             48, int(g["block_size"]))
    total = int(host(ws.num_tokens_post_padded)[0])
    assert total == g["expected_sorted"].size and total % 8 == 0
    assert np.array_equal(host(ws.sorted_token_ids)[:total], g["expected_sorted"])
    n = g["expected_expert_ids"].size
    assert np.array_equal(host(ws.expert_ids)[:n], g["expected_expert_ids"])
    assert routing.manifest_attrs()["sentinel_token_id"] == "56"


@pytest.mark.parametrize("tokens,bs,seed", [(1, 8, 0), (7, 8, 1), (64, 16, 2), (200, 32, 3),
                                            (300, 48, 4), (4096, 64, 5), (16384, 64, 6)])
def test_align_random_vs_oracle(oracle, tokens, bs, seed):
    g = np.random.default_rng(seed)
    gs = int(g.integers(0, 337))
    idx = g.integers(0, 384, size=(tokens, 8)).astype(np.int32)
    ws, _ = _gpu_align(idx, tokens, 8, gs, 48, bs)
    _check_against_oracle(oracle, ws, idx, gs, 48, bs)


def test_align_zipf_prefill_vs_oracle(oracle):
    from pegainfer_amd import synth
    idx, _ = synth.zipf_local_topk(synth.rng(5, 0), 4096)
    ws, _ = _gpu_align(idx, 4096, 8, 0, 48, 64)
    _check_against_oracle(oracle, ws, idx, 0, 48, 64)


def test_align_edge_cases(oracle):
    # no local routes at all
    idx = np.full((5, 8), 300, np.int32)
    ws, _ = _gpu_align(idx, 5, 8, 0, 48, 16)
    assert int(host(ws.num_tokens_post_padded)[0]) == 0
    assert (host(ws.sorted_token_ids) == 40).all() and (host(ws.expert_ids) == -1).all()
    _check_against_oracle(oracle, ws, idx, 0, 48, 16)
    # every route to one expert (maximum segment)
    idx = np.full((500, 8), 17, np.int32)
    ws, _ = _gpu_align(idx, 500, 8, 0, 48, 64)
    _check_against_oracle(oracle, ws, idx, 0, 48, 64)
    # capacity exactly at the bound routes + E*(bs-1)
    idx = np.arange(48 * 8, dtype=np.int32).reshape(48, 8) % 48
    ws, _ = _gpu_align(idx, 48, 8, 0, 48, 16)
    _check_against_oracle(oracle, ws, idx, 0, 48, 16)


@pytest.mark.parametrize("tokens", [255, 256, 257, 400, 511, 512, 513, 5000])
def test_align_wide_path_edges(oracle, tokens):
    """From 2048 routes the permutation runs one workgroup per expert (one
    launch below 4096 routes, two from there); these straddle both switches
    (255/256/257 and 511/512/513 tokens x top-8) and repeat the edge cases on
    each path."""
    g = np.random.default_rng(tokens)
    idx = g.integers(0, 384, size=(tokens, 8)).astype(np.int32)
    ws, _ = _gpu_align(idx, tokens, 8, 100, 48, 32)
    _check_against_oracle(oracle, ws, idx, 100, 48, 32)
    for fill, bs in ((300, 16), (17, 64)):  # no local route; every route to one expert
        idx = np.full((tokens, 8), fill, np.int32)
        ws, _ = _gpu_align(idx, tokens, 8, 0, 48, bs)
        _check_against_oracle(oracle, ws, idx, 0, 48, bs)
    # every expert present, routes in descending expert order
    idx = (47 - np.arange(tokens * 8, dtype=np.int32) % 48).reshape(tokens, 8)
    ws, _ = _gpu_align(idx, tokens, 8, 0, 48, 8)
    _check_against_oracle(oracle, ws, idx, 0, 48, 8)


@pytest.mark.parametrize("E,topk,tokens,bs", [(64, 6, 512, 64), (1, 1, 8, 8), (1, 1, 513, 64),
                                              (1, 1, 9000, 64), (512, 4, 2048, 8),
                                              (8, 8, 70000, 64),
                                              (224, 8, 100, 16), (512, 8, 3000, 32),
                                              (512, 4, 600, 8), (1, 1, 3000, 64),
                                              (37, 3, 70000, 48)])
def test_align_general_shapes(oracle, E, topk, tokens, bs):
    g = np.random.default_rng(E + topk)
    idx = g.integers(0, max(E, 2), size=(tokens, topk)).astype(np.int32)
    ws, _ = _gpu_align(idx, tokens, topk, 0, E, bs)
    _check_against_oracle(oracle, ws, idx, 0, E, bs)


def test_deepep_routing_vs_oracle(oracle):
    from pegainfer_amd import ops
    g = np.random.default_rng(3)
    E, align, bs = 48, 16, 16
    psum, cur = [], 0
    for c in g.integers(0, 40, size=E):
        cur = -(-cur // align) * align + int(c)
        psum.append(cur)
    psum.append(-(-cur // align) * align)
    ws = ops.KimiMarlinRouteWorkspace(512, bs)
    cap = psum[-1] + 64
    ops.kimi_deepep_build_marlin_routing_on_stream(ws, dev(np.array(psum, np.int32)), align, cap)
    ref = oracle.deepep_build_routing(np.array(psum, np.int32), E, align, bs, cap, -(-cap // bs))
    assert np.array_equal(host(ws.sorted_token_ids)[:cap], ref["sorted_token_ids"])
    assert np.array_equal(host(ws.expert_ids)[:-(-cap // bs)], ref["expert_ids"])
    assert int(host(ws.num_tokens_post_padded)[0]) == psum[-1]


@pytest.mark.parametrize("tokens,seed", [(1, 0), (64, 1), (4096, 2)])
def test_kimi_router_select_bit_exact(oracle, tokens, seed):
    from pegainfer_amd import ops
    g = np.random.default_rng(seed)
    logits = g.standard_normal((tokens, 384)).astype(np.float32)
    bias = (g.standard_normal(384) * 0.05).astype(np.float32) if seed else np.zeros(384, np.float32)
    w = torch.zeros(tokens, 8, dtype=torch.float32, device="cuda")
    idx = torch.zeros(tokens, 8, dtype=torch.int32, device="cuda")
    ops.kimi_router_select(dev(logits), dev(bias), w, idx, tokens)
    ref_idx, ref_w = oracle.kimi_router(logits, bias, 8, 1.0)
    assert np.array_equal(host(idx), ref_idx)
    assert np.array_equal(host(w), ref_w)


@pytest.mark.parametrize("tokens,seed", [(1, 0), (512, 1)])
def test_dsv2_router_select_bit_exact(oracle, tokens, seed):
    from pegainfer_amd import ops
    g = np.random.default_rng(seed)
    logits = g.standard_normal((tokens, 64)).astype(np.float32)
    if tokens > 1:
        logits[0] = load_golden("misc_kat.npz")["dsv2_logits"]
    w = torch.zeros(tokens, 6, dtype=torch.float32, device="cuda")
    idx = torch.zeros(tokens, 6, dtype=torch.int32, device="cuda")
    ops.dsv2_router_select(dev(logits), w, idx, tokens, 6)
    ref_idx, ref_w = oracle.dsv2_router(logits, 6)
    assert np.array_equal(host(idx), ref_idx)
    assert np.array_equal(host(w), ref_w)
    if tokens > 1:
        assert list(host(idx)[0]) == [7, 10, 20, 41, 54, 58]


@pytest.mark.parametrize("n_experts,topk", [(100, 4), (200, 8), (700, 8), (1024, 16)])
def test_kimi_router_select_expert_counts(oracle, n_experts, topk):
    from pegainfer_amd import ops
    g = np.random.default_rng(n_experts)
    tokens = 33
    logits = g.standard_normal((tokens, n_experts)).astype(np.float32)
    bias = (g.standard_normal(n_experts) * 0.05).astype(np.float32)
    w = torch.zeros(tokens, topk, dtype=torch.float32, device="cuda")
    idx = torch.zeros(tokens, topk, dtype=torch.int32, device="cuda")
    ops.kimi_router_select(dev(logits), dev(bias), w, idx, tokens, topk=topk)
    ref_idx, ref_w = oracle.kimi_router(logits, bias, topk, 1.0)
    assert np.array_equal(host(idx), ref_idx)
    assert np.array_equal(host(w), ref_w)


@pytest.mark.parametrize("active,padded,seed", [(64, 64, 0), (5, 64, 1), (1, 1, 2), (300, 320, 3)])
def test_kimi_router_noaux_tc_symbol(oracle, active, padded, seed):
    """kimi_k2_router_noaux_tc_cuda (ffi/kimi.rs:52-66): fp32 logits of every padded row
    within the fp32-accumulation bound of the oracle's (an fp64-free bound: K roundings
    of the running sum), then the select stage over the active rows bit for bit against
    the oracle fed the GPU's own logits; rows past active_tokens are not written."""
    from pegainfer_amd import ops, synth
    g = np.random.default_rng(40 + seed)
    H = 7168
    hidden = synth.normal_bf16(g, (padded, H))
    gate = synth.normal_bf16(g, (384, H), std=0.01)
    bias = (g.standard_normal(384) * 0.01).astype(np.float32)
    logits = torch.full((padded, 384), float("nan"), dtype=torch.float32, device="cuda")
    w = torch.full((padded, 8), -1.0, dtype=torch.float32, device="cuda")
    idx = torch.full((padded, 8), -5, dtype=torch.int32, device="cuda")
    ops.kimi_k2_router_noaux_tc(dev(hidden), dev(gate), dev(bias), logits, w, idx, active, padded)
    got_l = host(logits)
    ref_l = oracle.dense_gemm_f32(gate, hidden)
    hf = oracle.bf16_to_f32(hidden).astype(np.float64)
    gf = oracle.bf16_to_f32(gate).astype(np.float64)
    bound = 2 * H * 2.0 ** -24 * (np.abs(hf) @ np.abs(gf).T)  # both sums' rounding errors
    assert np.isfinite(got_l).all()
    assert (np.abs(got_l.astype(np.float64) - ref_l) <= bound).all()
    ref_idx, ref_w = oracle.kimi_router(got_l[:active], bias, 8, 1.0)
    assert np.array_equal(host(idx)[:active], ref_idx)
    assert np.array_equal(host(w)[:active], ref_w)
    assert (host(idx)[active:] == -5).all() and (host(w)[active:] == -1.0).all()
    # the oracle's own logits pick the same experts where the margin is clear
    m = synth.kimi_topk_margin(ref_l[:active], bias)
    ok = m > 1e-4
    assert ok.mean() > 0.9
    ref_idx2, _ = oracle.kimi_router(ref_l[:active], bias, 8, 1.0)
    assert np.array_equal(ref_idx2[ok], ref_idx[ok])


@pytest.mark.parametrize("tokens,bs,start,n_experts,E,seed", [
    (1, 8, 0, 384, 48, 0), (3, 8, 48, 384, 48, 1), (16, 16, 0, 384, 48, 2),
    (64, 16, 96, 384, 48, 3), (200, 32, 0, 384, 48, 4), (512, 64, 336, 384, 48, 5),
    (64, 16, 0, 64, 64, 6), (37, 8, 10, 200, 17, 7), (24, 16, 0, 384, 48, 8),
    (40, 16, 0, 1000, 48, 9), (100, 32, 0, 1024, 64, 10)])
def test_kimi_route_align_matches_two_launches(oracle, tokens, bs, start, n_experts, E, seed):
    """The fused select + permutation (one workgroup) against the select kernel followed
    by the permutation kernel: top-k ids and weights and every routing array bit for
    bit, and the permutation against the oracle; outputs past the active rows and
    the routing capacity are left as they were."""
    from pegainfer_amd import ops
    g = np.random.default_rng(70 + seed)
    logits = dev(g.standard_normal((tokens, n_experts)).astype(np.float32))
    bias = dev((g.standard_normal(n_experts) * 0.02).astype(np.float32))
    ws_a = ops.KimiMarlinRouteWorkspace(tokens + 5, bs, topk=8, local_experts=E)
    ws_b = ops.KimiMarlinRouteWorkspace(tokens + 5, bs, topk=8, local_experts=E)
    for ws in (ws_a, ws_b):
        for t in (ws.sorted_token_ids, ws.expert_ids, ws.expert_offsets, ws.expert_cursor):
            t.fill_(-7)
    w_a = torch.full(((tokens + 5) * 8,), -1.0, dtype=torch.float32, device="cuda")
    w_b = w_a.clone()
    i_a = torch.full(((tokens + 5) * 8,), -3, dtype=torch.int32, device="cuda")
    i_b = i_a.clone()
    ops.kimi_router_select(logits, bias, w_a, i_a, tokens)
    ops.moe_align_block_size(ws_a, i_a, tokens, tokens, start)
    ops.kimi_route_align(ws_b, logits, bias, w_b, i_b, tokens, start)
    torch.cuda.synchronize()
    assert np.array_equal(host(i_a), host(i_b))
    assert np.array_equal(host(w_a).view(np.uint32), host(w_b).view(np.uint32))
    assert (host(i_b)[tokens * 8:] == -3).all() and (host(w_b)[tokens * 8:] == -1.0).all()
    for name in ("sorted_token_ids", "expert_ids", "num_tokens_post_padded", "expert_offsets",
                 "expert_cursor"):
        assert np.array_equal(host(getattr(ws_a, name)), host(getattr(ws_b, name))), name
    _check_against_oracle(oracle, ws_b, host(i_b)[:tokens * 8], start, E, bs)


def test_kimi_route_align_rejections():
    """Argument checks of the fused entry point: the select's and the permutation's
    (status 1), and more than 4096 routes (801), all before any launch."""
    from pegainfer_amd import _lib, ops
    ws = ops.KimiMarlinRouteWorkspace(600, 64, topk=8, local_experts=48)
    logits = torch.zeros(600, 384, dtype=torch.float32, device="cuda")
    bias = torch.zeros(384, dtype=torch.float32, device="cuda")
    w = torch.zeros(600 * 8, dtype=torch.float32, device="cuda")
    i = torch.zeros(600 * 8, dtype=torch.int32, device="cuda")
    L = _lib.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    base = [P(logits), P(bias), P(w), P(i), P(ws.sorted_token_ids), P(ws.expert_ids),
            P(ws.num_tokens_post_padded), P(ws.expert_offsets), P(ws.expert_cursor)]

    def call(tokens, n_experts=384, topk=8, scale=1.0, start=0, E=48, bs=64,
             padded=ws.max_padded_tokens, blocks=ws.max_m_blocks):
        return L.pega_kimi_route_align(*base, tokens, n_experts, topk, ctypes.c_float(scale),
                                       start, E, bs, padded, blocks, None)
    assert call(513) == 801                       # 4104 routes
    assert call(0) == 1 and call(4, topk=0) == 1 and call(4, scale=0.0) == 1
    assert call(4, n_experts=1025) == 1 and call(4, E=513) == 1 and call(4, bs=24) == 1
    assert call(4, padded=10) == 1 and call(4, blocks=0) == 1
    base[0] = ctypes.c_void_p(0)
    assert call(4) == 1



@pytest.mark.parametrize("tokens,bs,start,E,seed", [
    (1, 8, 0, 64, 0), (4, 16, 0, 64, 1), (5, 16, 8, 48, 2), (64, 32, 0, 64, 3),
    (512, 64, 0, 64, 4), (682, 64, 0, 64, 5), (100, 64, 16, 32, 6)])
def test_dsv2_route_align_matches_two_launches(oracle, tokens, bs, start, E, seed):
    """The fused DeepSeek-V2-Lite select + permutation against the select kernel followed
    by the permutation kernel (64 experts, top-6), bit for bit, and the permutation against
    the oracle; outputs past the active rows are left as they were."""
    from pegainfer_amd import ops
    g = np.random.default_rng(170 + seed)
    logits = dev(g.standard_normal((tokens, 64)).astype(np.float32))
    ws_a = ops.KimiMarlinRouteWorkspace(tokens + 3, bs, topk=6, local_experts=E)
    ws_b = ops.KimiMarlinRouteWorkspace(tokens + 3, bs, topk=6, local_experts=E)
    for ws in (ws_a, ws_b):
        for t in (ws.sorted_token_ids, ws.expert_ids, ws.expert_offsets, ws.expert_cursor):
            t.fill_(-7)
    w_a = torch.full(((tokens + 3) * 6,), -1.0, dtype=torch.float32, device="cuda")
    w_b = w_a.clone()
    i_a = torch.full(((tokens + 3) * 6,), -3, dtype=torch.int32, device="cuda")
    i_b = i_a.clone()
    ops.dsv2_router_select(logits, w_a, i_a, tokens, 6)
    ops.moe_align_block_size(ws_a, i_a, tokens, tokens, start)
    ops.dsv2_route_align(ws_b, logits, w_b, i_b, tokens, start)
    torch.cuda.synchronize()
    assert np.array_equal(host(i_a), host(i_b))
    assert np.array_equal(host(w_a).view(np.uint32), host(w_b).view(np.uint32))
    assert (host(i_b)[tokens * 6:] == -3).all() and (host(w_b)[tokens * 6:] == -1.0).all()
    for name in ("sorted_token_ids", "expert_ids", "num_tokens_post_padded", "expert_offsets",
                 "expert_cursor"):
        assert np.array_equal(host(getattr(ws_a, name)), host(getattr(ws_b, name))), name
    _check_against_oracle(oracle, ws_b, host(i_b)[:tokens * 6], start, E, bs)


@pytest.mark.parametrize("tokens", [1, 4, 64, 512])
def test_fused_route_align_against_the_oracle_routers(oracle, tokens):
    """Both fused entry points straight against the CPU routers (oracle.kimi_router,
    oracle.dsv2_router): ids and weights bit for bit, and the permutation of those ids."""
    from pegainfer_amd import ops
    g = np.random.default_rng(300 + tokens)
    # Kimi: 384 experts, top-8, nonzero bias, 48 local experts from 96
    logits = g.standard_normal((tokens, 384)).astype(np.float32)
    bias = (g.standard_normal(384) * 0.03).astype(np.float32)
    ws = ops.KimiMarlinRouteWorkspace(tokens, 16, topk=8, local_experts=48)
    w = torch.zeros(tokens * 8, dtype=torch.float32, device="cuda")
    i = torch.zeros(tokens * 8, dtype=torch.int32, device="cuda")
    ops.kimi_route_align(ws, dev(logits), dev(bias), w, i, tokens, 96, route_scale=2.5)
    ref_idx, ref_w = oracle.kimi_router(logits, bias, 8, 2.5)
    assert np.array_equal(host(i).reshape(tokens, 8), ref_idx)
    assert np.array_equal(host(w).reshape(tokens, 8).view(np.uint32), ref_w.view(np.uint32))
    _check_against_oracle(oracle, ws, ref_idx.reshape(-1), 96, 48, 16)
    # DeepSeek-V2-Lite: 64 experts, top-6 softmax, all local
    logits = g.standard_normal((tokens, 64)).astype(np.float32)
    if tokens >= 4:
        logits[3] = load_golden("misc_kat.npz")["dsv2_logits"]
    ws = ops.KimiMarlinRouteWorkspace(tokens, 64, topk=6, local_experts=64)
    w = torch.zeros(tokens * 6, dtype=torch.float32, device="cuda")
    i = torch.zeros(tokens * 6, dtype=torch.int32, device="cuda")
    ops.dsv2_route_align(ws, dev(logits), w, i, tokens, 0)
    ref_idx, ref_w = oracle.dsv2_router(logits, 6)
    assert np.array_equal(host(i).reshape(tokens, 6), ref_idx)
    assert np.array_equal(host(w).reshape(tokens, 6).view(np.uint32), ref_w.view(np.uint32))
    if tokens >= 4:
        assert list(ref_idx[3]) == [7, 10, 20, 41, 54, 58]
    _check_against_oracle(oracle, ws, ref_idx.reshape(-1), 0, 64, 64)


def test_fused_route_align_repeated_and_graph_replays():
    """The multi-workgroup hand-off resets its arrival counter: calls in a row with
    different token counts, then a captured call replayed with new logits copied in
    between (eager work and synchronisation between replays), each equal to the two
    launches."""
    from pegainfer_amd import layer, ops
    g = np.random.default_rng(5)
    T = 64
    logits = torch.zeros(T, 384, dtype=torch.float32, device="cuda")
    bias = dev((g.standard_normal(384) * 0.02).astype(np.float32))
    ws_a = ops.KimiMarlinRouteWorkspace(T, 16, topk=8, local_experts=48)
    ws_b = ops.KimiMarlinRouteWorkspace(T, 16, topk=8, local_experts=48)
    w_a = torch.zeros(T * 8, dtype=torch.float32, device="cuda")
    i_a = torch.zeros(T * 8, dtype=torch.int32, device="cuda")
    w_b, i_b = w_a.clone(), i_a.clone()

    def compare(n):
        ops.kimi_router_select(logits, bias, w_a, i_a, n)
        ops.moe_align_block_size(ws_a, i_a, n, n, 0)
        torch.cuda.synchronize()
        assert np.array_equal(host(i_a)[:n * 8], host(i_b)[:n * 8])
        assert np.array_equal(host(w_a)[:n * 8], host(w_b)[:n * 8])
        for name in ("sorted_token_ids", "expert_ids", "num_tokens_post_padded",
                     "expert_offsets", "expert_cursor"):
            assert np.array_equal(host(getattr(ws_a, name)), host(getattr(ws_b, name))), name

    for n in (64, 9, 64, 33, 5, 64):
        logits.copy_(dev(g.standard_normal((T, 384)).astype(np.float32)))
        ops.kimi_route_align(ws_b, logits, bias, w_b, i_b, n, 0)
        compare(n)
    graph = layer.capture_graph(lambda: ops.kimi_route_align(ws_b, logits, bias, w_b, i_b, T, 0))
    for _ in range(3):
        logits.copy_(dev(g.standard_normal((T, 384)).astype(np.float32)))
        torch.cuda.synchronize()
        graph.replay()
        compare(T)


def test_router_exp_equals_double_exp_over_every_float():
    """The routers' e^x (exp_exact_f32_fast through pega_exp_exact_f32: a double polynomial
    that falls back to the double exp within 2^-45 of an fp32 rounding midpoint) equals the
    device's double-precision exp rounded to fp32 (torch's float64 exp, the same device
    library) at every float with |x| <= 80 -- about 2.2e9 values, subnormals and both zeros
    included -- and at the values outside that range, which take the fallback."""
    from pegainfer_amd import _lib
    from pegainfer_amd.ops import _ptr, _stream
    top = int(np.array([80.0], np.float32).view(np.int32)[0])
    chunk = 1 << 27
    y = torch.empty(chunk, dtype=torch.float32, device="cuda")
    checked = 0
    for sign in (0, -(1 << 31)):
        for lo in range(0, top + 1, chunk):
            hi = min(lo + chunk, top + 1)
            bits = (torch.arange(lo, hi, dtype=torch.int64, device="cuda") + sign).to(torch.int32)
            x = bits.view(torch.float32)
            _lib.call("pega_exp_exact_f32", _ptr(x), _ptr(y), hi - lo, _stream())
            want = torch.exp(x.double()).float()
            got = y[:hi - lo]
            bad = (got.view(torch.int32) != want.view(torch.int32)).sum().item()
            assert bad == 0, f"{bad} mismatches in [{lo:#x}, {hi:#x}) sign {sign}"
            checked += hi - lo
    assert checked > 2_200_000_000
    outside = torch.tensor([80.5, -80.5, 88.7, 89.0, -103.0, -104.0, 1e30, -1e30,
                            float("inf"), float("-inf")], dtype=torch.float32, device="cuda")
    out = torch.empty_like(outside)
    _lib.call("pega_exp_exact_f32", _ptr(outside), _ptr(out), outside.numel(), _stream())
    assert torch.equal(out.view(torch.int32), torch.exp(outside.double()).float().view(torch.int32))
    nan = torch.tensor([float("nan")], dtype=torch.float32, device="cuda")
    _lib.call("pega_exp_exact_f32", _ptr(nan), _ptr(out), 1, _stream())
    assert torch.isnan(out[0]).item()

