"""GPU parity of the grouped W4A16 GEMM (K2) against the oracle.

Exact cases (power-of-two scales with small-integer activations, one-hot
rows) must match bit for bit whatever the summation order; random cases are
held to the BASELINE tolerance |gpu - ref| <= 1e-3 + 1e-2 |ref|.  Both the
decode kernel (block sizes 8/16, split-K) and the prefill kernel (32/48/64,
128-row tiles) are exercised, through the reference-shaped entry point (48
experts) and the shape-general one.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_bf16_close, dev, host, pack_ckpt

pytestmark = pytest.mark.gpu


def _setup(E, N, K, q, scale_bits, device="cuda"):
    from pegainfer_amd import ops
    packed = pack_ckpt(q)
    w = ops.marlin_int4_reorder(dev(packed.reshape(-1)), dev(scale_bits.reshape(-1)), E, K, N)
    return w, packed


def _run(oracle, *, E, N, K, T, topk, bs, mul, a_bits, q, scale_bits, idx, tw, global_start=0,
         extra_splits=1, poison=True, threads=8, repeat=1):
    from pegainfer_amd import ops
    w, packed = _setup(E, N, K, q, scale_bits)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx.reshape(-1).astype(np.int32)), T, T,
                                       global_start)
    gws = ops.KimiMarlinWna16Workspace(ws.max_m_blocks, N, bs, extra_splits=extra_splits)
    out = torch.full((T * topk, N), 7.0 if poison else 0.0, dtype=torch.bfloat16, device="cuda")
    a = dev(a_bits)
    twd = dev(tw.reshape(-1).astype(np.float32))
    for _ in range(repeat):
        ops.wna16_gemm(gws, routing, a, w, twd, out, top_k=topk, mul_topk_weights=mul, size_m=T)
    got = host(out)
    assert (host(gws.locks) == 0).all(), "locks must be left at zero"
    ref_routing = {k: host(v) for k, v in (("sorted_token_ids", routing.sorted_token_ids),
                                           ("expert_ids", routing.expert_ids),
                                           ("num_tokens_post_padded", routing.num_tokens_post_padded))}
    init = np.full((T * topk, N), 0x40E0 if poison else 0, np.uint16)  # bf16(7.0)
    ref = oracle.wna16_gemm(a_bits, packed, scale_bits, ref_routing, tw, moe_block_size=bs,
                            top_k=topk, mul_topk_weights=mul, size_m=T, size_n=N, size_k=K,
                            output=init, threads=threads)
    return got, ref


@pytest.mark.parametrize("bs", [16, 64])
def test_gemm_exact_small_integers(oracle, bs):
    g = np.random.default_rng(bs)
    E, N, K, T = 3, 128, 512, 40
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(np.ldexp(1.0, g.integers(-6, 2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-4, 5, size=(T, K)).astype(np.float32))
    idx = g.integers(0, E, size=(T, 1))
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=1, bs=bs, mul=False, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=np.ones((T, 1), np.float32))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("bs", [16, 64])
def test_gemm_one_hot_rows_give_dequantised_weights(oracle, bs):
    g = np.random.default_rng(100 + bs)
    E, N, K = 2, 192, 64
    T = K
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16((np.abs(g.standard_normal((E, N, K // 32))) * 0.013).astype(np.float32))
    a_bits = oracle.f32_to_bf16(np.eye(K, dtype=np.float32))
    idx = np.ones((T, 1), np.int64)  # all rows to expert 1
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=1, bs=bs, mul=False, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=np.ones((T, 1), np.float32))
    assert np.array_equal(got, ref)
    s = (scale_bits.astype(np.uint32) << 16).view(np.float32)
    want = oracle.f32_to_bf16((q[1] * np.repeat(s[1], 32, axis=1)).astype(np.float32)).T
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bs,topk,mul,T", [(8, 8, False, 5), (16, 8, False, 64), (16, 1, True, 512),
                                           (32, 8, False, 150), (48, 8, True, 230),
                                           (64, 8, False, 700), (64, 1, True, 2000)])
def test_gemm_random_kimi_entry(oracle, bs, topk, mul, T):
    """48 local experts through kimi_marlin_wna16_gemm_cuda (reduced N, K)."""
    g = np.random.default_rng(bs * 31 + T)
    E, N, K = 48, 256, 512
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16((np.abs(g.standard_normal((E, N, K // 32))) * 0.02 / 7).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.standard_normal((T, K)).astype(np.float32))
    idx = g.integers(0, 96, size=(T, topk))  # about half the routes are local
    tw = g.random((T, topk)).astype(np.float32)
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=topk, bs=bs, mul=mul, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=tw, global_start=24)
    untouched = ref == 0x40E0
    assert np.array_equal(got[untouched], ref[untouched])  # rows not routed here keep their value
    assert_bf16_close(got, ref, what=f"bs={bs} topk={topk} mul={mul}")


@pytest.mark.parametrize("rows,N,K,splits", [(1, 9728, 2560, 8), (4, 4096, 7168, 8),
                                             (8, 7168, 2048, 8), (3, 512, 1024, 1)])
def test_gemm_dense_split_k(oracle, rows, N, K, splits):
    """One expert (C1/C2 shapes) through the shape-general entry, whose c_tmp
    may be larger than the reference's (`splits`); called twice, and the lock
    workspace is never written."""
    g = np.random.default_rng(rows * 7 + N)
    q = g.integers(-8, 8, size=(1, N, K))
    scale_bits = oracle.f32_to_bf16((np.abs(g.standard_normal((1, N, K // 32))) * 0.02 / 7).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.standard_normal((rows, K)).astype(np.float32))
    got, ref = _run(oracle, E=1, N=N, K=K, T=rows, topk=1, bs=8 if rows <= 8 else 16, mul=False,
                    a_bits=a_bits, q=q, scale_bits=scale_bits, idx=np.zeros((rows, 1)),
                    tw=np.ones((rows, 1), np.float32), extra_splits=splits, repeat=2)
    assert_bf16_close(got, ref, what=f"dense rows={rows} N={N} K={K}")


def test_gemm_deterministic_across_runs(oracle):
    g = np.random.default_rng(5)
    E, N, K, T = 48, 256, 1024, 64
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16((np.abs(g.standard_normal((E, N, K // 32))) * 0.01).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.standard_normal((T, K)).astype(np.float32))
    idx = g.integers(0, 48, size=(T, 8))
    outs = []
    for _ in range(2):
        got, _ = _run(oracle, E=E, N=N, K=K, T=T, topk=8, bs=16, mul=False, a_bits=a_bits, q=q,
                      scale_bits=scale_bits, idx=idx, tw=np.ones((T, 8), np.float32))
        outs.append(got)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("rows,N,K", [(1, 9728, 2560), (8, 4096, 7168)])
def test_gemm_small_batch_exact_and_deterministic(oracle, rows, N, K):
    """Decode of one expert at a small batch (16 waves split K inside each
    workgroup) on a case whose every partial sum is exact (small-integer
    activations, power-of-two scales): bit-exact with the oracle, and
    identical across calls.  Also a regression test for a wrong-result bug in
    the bs <= 8 decode variant: a dequant step written as a vector inline-asm
    statement hid a register write from the compiler's MFMA hazard tracking,
    and it landed in an MFMA destination still in flight."""
    g = np.random.default_rng(rows + K)
    q = g.integers(-8, 8, size=(1, N, K))
    scale_bits = oracle.f32_to_bf16(
        (2.0 ** g.integers(-6, -2, size=(1, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-2, 3, size=(rows, K)).astype(np.float32))
    outs = []
    for _ in range(2):
        got, ref = _run(oracle, E=1, N=N, K=K, T=rows, topk=1, bs=8, mul=False, a_bits=a_bits,
                        q=q, scale_bits=scale_bits, idx=np.zeros((rows, 1)),
                        tw=np.ones((rows, 1), np.float32), extra_splits=8)
        assert np.array_equal(got, ref)
        outs.append(got)
    assert np.array_equal(outs[0], outs[1])


def test_gemm_block8_four_waves_exact(oracle):
    """Block size 8 with enough workgroups that 4 waves split K (the bs <= 8,
    4-wave decode variant, main prefetch loop included: 20 groups per wave),
    48 experts through the reference entry, exact inputs: bit-exact.  This is
    the configuration in which the inline-asm hazard above corrupted the
    n0 columns."""
    g = np.random.default_rng(77)
    E, N, K, T = 48, 2048, 2560, 8
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(
        (2.0 ** g.integers(-6, -2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-2, 3, size=(T, K)).astype(np.float32))
    idx = g.integers(0, 48, size=(T, 8))
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=8, bs=8, mul=False, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=np.ones((T, 8), np.float32), threads=16)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("E,T,topk,bs,inter,K,split_k", [
    (1, 1, 1, 8, 2048, 7168, True), (1, 8, 1, 8, 1024, 2048, True), (48, 4, 8, 16, 512, 1024, True),
    (1, 1, 1, 8, 2048, 7168, False), (1, 8, 1, 8, 1024, 2048, False),
    (48, 4, 8, 16, 512, 1024, False), (48, 64, 8, 16, 512, 1024, True),
    (3, 300, 4, 32, 192, 256, True), (48, 160, 8, 48, 1024, 512, True),
    (4, 512, 2, 64, 1408, 256, True)])
def test_w13_swiglu_fused_exact(oracle, E, T, topk, bs, inter, K, split_k):
    """pega_wna16_w13_swiglu on exact inputs: every W13 value is exact, so the
    activations equal oracle SwiGLU(oracle W13) bit for bit; rows of routes that are
    not local keep their contents.  Block sizes 8/16 split K across workgroups when the
    units are few (partials summed and rounded by the SwiGLU kernel) and otherwise, or
    with split_k=False, pair each gate tile with its up tile in one workgroup (SwiGLU in
    the epilogue; the 48-expert, 64-token case picks that path by itself); 32/48/64 take
    the tile GEMM with the SwiGLU epilogue (an odd gate-tile count leaves a workgroup half
    its columns)."""
    from pegainfer_amd import ops
    g = np.random.default_rng(E * 100 + T)
    N = 2 * inter
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(
        (2.0 ** g.integers(-6, -2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-2, 3, size=(T, K)).astype(np.float32))
    idx = g.integers(0, 2 * E, size=(T, topk)).astype(np.int32)  # about half not local
    w, packed = _setup(E, N, K, q, scale_bits)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx.reshape(-1)), T, T, 0)
    gws = ops.KimiMarlinWna16Workspace(ws.max_m_blocks, N, bs, extra_splits=16)
    act = torch.full((T * topk, inter), 3.0, dtype=torch.bfloat16, device="cuda")
    for _ in range(2):
        ops.wna16_w13_swiglu(gws, routing, dev(a_bits), w, act, top_k=topk, size_m=T,
                             split_k=split_k)
    got = host(act)
    r = {k: host(v) for k, v in (("sorted_token_ids", routing.sorted_token_ids),
                                 ("expert_ids", routing.expert_ids),
                                 ("num_tokens_post_padded", routing.num_tokens_post_padded))}
    ref13 = oracle.wna16_gemm(a_bits, packed, scale_bits, r, np.ones((T, topk), np.float32),
                              moe_block_size=bs, top_k=topk, mul_topk_weights=False, size_m=T,
                              size_n=N, size_k=K, threads=16)
    local = (idx.reshape(-1) < E)
    assert np.array_equal(got[local], oracle.swiglu(ref13, inter)[local])
    assert (got[~local] == 0x4040).all()  # bf16(3.0) untouched


@pytest.mark.parametrize("seed", range(40))
def test_gemm_and_w13_swiglu_shape_sweep_exact(oracle, seed):
    """Seeded random shapes through both kernels: experts 1-20, tokens 1-400, top-k 1-8,
    every block size, N and K from one to several tiles (odd chunk and gate-tile counts
    included), with and without the top-k weight.  Inputs are exact (small-integer
    activations, power-of-two scales), so every sum is exact and both the GEMM output
    and W13 + SwiGLU must equal the oracle bit for bit; rows not routed here keep
    their contents."""
    from pegainfer_amd import ops
    g = np.random.default_rng(900 + seed)
    bs = int(g.choice([8, 16, 32, 48, 64]))
    E = int(g.integers(1, 21))
    T = int(g.integers(1, 401))
    topk = int(min(g.choice([1, 2, 6, 8]), 2 * E))
    K = 64 * int(g.integers(1, 11))
    inter = 64 * int(g.integers(1, 6))
    N = 2 * inter
    mul = bool(g.integers(0, 2))
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(
        (2.0 ** g.integers(-6, -2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-2, 3, size=(T, K)).astype(np.float32))
    idx = np.stack([g.permutation(2 * E)[:topk] for _ in range(T)]).astype(np.int32)
    tw = oracle.bf16_to_f32(oracle.f32_to_bf16(g.random((T, topk)).astype(np.float32)))
    what = f"seed={seed} bs={bs} E={E} T={T} topk={topk} N={N} K={K} mul={mul}"
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=topk, bs=bs, mul=mul, a_bits=a_bits,
                    q=q, scale_bits=scale_bits, idx=idx, tw=tw, extra_splits=4)
    assert np.array_equal(got, ref), what
    w, packed = _setup(E, N, K, q, scale_bits)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx.reshape(-1)), T, T, 0)
    gws = ops.KimiMarlinWna16Workspace(ws.max_m_blocks, N, bs, extra_splits=16)
    act = torch.full((T * topk, inter), 3.0, dtype=torch.bfloat16, device="cuda")
    ops.wna16_w13_swiglu(gws, routing, dev(a_bits), w, act, top_k=topk, size_m=T)
    r = {k: host(v) for k, v in (("sorted_token_ids", routing.sorted_token_ids),
                                 ("expert_ids", routing.expert_ids),
                                 ("num_tokens_post_padded", routing.num_tokens_post_padded))}
    ref13 = oracle.wna16_gemm(a_bits, packed, scale_bits, r, np.ones((T, topk), np.float32),
                              moe_block_size=bs, top_k=topk, mul_topk_weights=False, size_m=T,
                              size_n=N, size_k=K, threads=16)
    local = idx.reshape(-1) < E
    got_act = host(act)
    assert np.array_equal(got_act[local], oracle.swiglu(ref13, inter)[local]), what
    assert (got_act[~local] == 0x4040).all(), what


def test_prefill_tile_scan_runs_and_gaps(oracle):
    """Prefill tiles found by the block-expert scan: an expert with two separate
    runs, runs shorter and longer than a tile, and blocks of expert -1 holding
    real token ids (their rows must stay untouched)."""
    from types import SimpleNamespace
    from pegainfer_amd import ops
    g = np.random.default_rng(11)
    E, N, K, bs = 3, 128, 256, 32  # 32-row blocks: prefill kernel, 4 blocks per tile
    runs = [(0, 3), (-1, 1), (1, 5), (0, 2), (2, 1), (-1, 2), (1, 4)]
    nblocks = sum(n for _, n in runs)
    T = nblocks * bs
    expert_ids, sorted_ids, tok = [], [], 0
    for e, n in runs:
        for b in range(n):
            expert_ids.append(e)
            for r in range(bs):
                if e >= 0 and b == n - 1 and r >= bs - 5:
                    sorted_ids.append(T)  # padding at the end of a run
                else:
                    sorted_ids.append(tok)
                    tok += 1
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(np.ldexp(1.0, g.integers(-6, 2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-4, 5, size=(T, K)).astype(np.float32))
    w, packed = _setup(E, N, K, q, scale_bits)
    st, ei = np.array(sorted_ids, np.int32), np.array(expert_ids, np.int32)
    ntp = np.array([nblocks * bs], np.int32)
    routing = SimpleNamespace(block_size=bs, max_m_blocks=nblocks, max_padded_tokens=nblocks * bs,
                              sorted_token_ids=dev(st), expert_ids=dev(ei),
                              num_tokens_post_padded=dev(ntp))
    gws = ops.KimiMarlinWna16Workspace(nblocks, N, bs)
    out = torch.full((T, N), 7.0, dtype=torch.bfloat16, device="cuda")
    tw = np.ones((T, 1), np.float32)
    ops.wna16_gemm(gws, routing, dev(a_bits), w, dev(tw.reshape(-1)), out, top_k=1,
                   mul_topk_weights=False, size_m=T)
    got = host(out)
    ref = oracle.wna16_gemm(a_bits, packed, scale_bits,
                            {"sorted_token_ids": st, "expert_ids": ei, "num_tokens_post_padded": ntp},
                            tw, moe_block_size=bs, top_k=1, mul_topk_weights=False, size_m=T,
                            size_n=N, size_k=K, output=np.full((T, N), 0x40E0, np.uint16), threads=8)
    assert np.array_equal(got, ref)
    gap_rows = [sorted_ids[b * bs + r] for b, e in enumerate(expert_ids) if e < 0 for r in range(bs)]
    assert (got[gap_rows] == 0x40E0).all(), "rows of expert -1 blocks must stay untouched"


def test_prefill_tile_scan_over_many_blocks(oracle):
    """More than 1024 m-blocks: the tile scan stages the block experts in
    several passes."""
    g = np.random.default_rng(12)
    E, N, K, T, topk, bs = 8, 64, 64, 4400, 8, 32
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(np.ldexp(1.0, g.integers(-6, 2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-4, 5, size=(T, K)).astype(np.float32))
    idx = np.stack([g.permutation(E) for _ in range(T)]).astype(np.int32)  # every token to every expert
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=topk, bs=bs, mul=False, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=np.ones((T, topk), np.float32))
    routes = int((idx < E).sum())
    assert routes // bs > 1024, "the case must span more than one scan slab"
    assert np.array_equal(got, ref)


def _pair_problem(g, oracle, *, E, T, topk, bs, N, K, swiglu, mul, none_local=False):
    """Random problem (weights, routing, poisoned output) for the pair entry;
    none_local: every route belongs to another GPU (no tile at all)."""
    from pegainfer_amd import ops
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16((2.0 ** g.integers(-7, -3, size=(E, N, K // 32))).astype(np.float32))
    w, _ = _setup(E, N, K, q, scale_bits)
    a = dev(oracle.f32_to_bf16(g.standard_normal((T, K)).astype(np.float32)))
    idx = g.integers(0, 2 * E if E > 1 else 1, size=(T, topk)).astype(np.int32)
    if none_local:
        idx = idx % E + E
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx.reshape(-1)), T, T, 0)
    tw = dev(g.random((T, topk)).astype(np.float32))
    width = N // 2 if swiglu else N
    outs = [torch.full((T * topk, width), 5.0, dtype=torch.bfloat16, device="cuda")
            for _ in range(2)]
    return dict(ws=ws, routing=routing, w=w, a=a, tw=tw, outs=outs, T=T, topk=topk, bs=bs, N=N,
                swiglu=swiglu, mul=mul)


def _single_launch(pr, out):
    from pegainfer_amd import ops
    gws = ops.KimiMarlinWna16Workspace(pr["ws"].max_m_blocks, pr["N"], pr["bs"])
    if pr["swiglu"]:
        ops.wna16_w13_swiglu(gws, pr["routing"], pr["a"], pr["w"], out, top_k=pr["topk"],
                             size_m=pr["T"])
    else:
        ops.wna16_gemm(gws, pr["routing"], pr["a"], pr["w"], pr["tw"], out, top_k=pr["topk"],
                       mul_topk_weights=pr["mul"], size_m=pr["T"])


def _pair_struct(pr, out):
    from pegainfer_amd import ops
    kw = dict(act=out) if pr["swiglu"] else dict(output=out, topk_weight=pr["tw"],
                                                 mul_topk_weights=pr["mul"])
    return ops.wna16_problem(pr["routing"], pr["a"], pr["w"], top_k=pr["topk"], size_m=pr["T"],
                             **kw)


@pytest.mark.parametrize("first,second", [
    # a shared expert's W13 + SwiGLU (one expert, every row) with routed W13 + SwiGLU
    (dict(E=1, T=512, topk=1, bs=64, N=2 * 704, K=512, swiglu=True, mul=False),
     dict(E=16, T=512, topk=6, bs=64, N=2 * 192, K=512, swiglu=True, mul=False)),
    # shared W2 (long K) with routed W2 times the top-k weight
    (dict(E=1, T=300, topk=1, bs=64, N=512, K=1024, swiglu=False, mul=False),
     dict(E=8, T=300, topk=4, bs=32, N=512, K=256, swiglu=False, mul=True)),
    # mixed kinds and block sizes, more workgroups in the first problem
    (dict(E=5, T=200, topk=3, bs=48, N=1024, K=256, swiglu=False, mul=True),
     dict(E=3, T=40, topk=2, bs=32, N=2 * 128, K=768, swiglu=True, mul=False)),
    # one problem without a single local route: its workgroups all leave at once
    (dict(E=4, T=64, topk=2, bs=32, N=512, K=512, swiglu=False, mul=False, none_local=True),
     dict(E=6, T=100, topk=4, bs=64, N=2 * 256, K=512, swiglu=True, mul=False)),
    (dict(E=1, T=128, topk=1, bs=64, N=2 * 192, K=256, swiglu=True, mul=False),
     dict(E=8, T=50, topk=8, bs=32, N=256, K=256, swiglu=False, mul=True, none_local=True)),
])
def test_prefill_pair_matches_single_launches(oracle, first, second):
    """pega_wna16_prefill_pair runs both problems in one launch; each output has the
    bits of its own single launch (pega_wna16_gemm / pega_wna16_w13_swiglu), and rows
    of routes that are not local keep their contents."""
    from pegainfer_amd import ops
    g = np.random.default_rng(first["N"] + second["K"])
    p0 = _pair_problem(g, oracle, **first)
    p1 = _pair_problem(g, oracle, **second)
    for pr in (p0, p1):
        _single_launch(pr, pr["outs"][0])
    s0, s1 = _pair_struct(p0, p0["outs"][1]), _pair_struct(p1, p1["outs"][1])
    ops.wna16_prefill_pair(s0, s1)
    ops.wna16_prefill_pair(s0, s1)  # a replay writes the same values
    for pr, spec in ((p0, first), (p1, second)):
        ref, got = host(pr["outs"][0]), host(pr["outs"][1])
        assert np.array_equal(got, ref)
        if spec.get("none_local"):
            assert (got == 0x40A0).all(), "no local route: nothing is written"
            continue
        assert (ref != 0x40A0).any()
        if spec["E"] > 1:
            assert (ref == 0x40A0).all(axis=1).any(), "rows of other GPUs' routes keep bf16(5.0)"


@pytest.mark.parametrize("bs", [32, 48, 64])
@pytest.mark.parametrize("swiglu", [False, True])
def test_prefill_tile_heights_agree(oracle, bs, swiglu):
    """The prefill kernel runs 64-row tiles when the routes could fill at most 64 rows
    per expert and 128-row tiles otherwise; every output's sum is the same MFMA sequence
    in either.  The tile height follows (routes, expert count), so the same problem goes
    through the shape-general entries with its real expert count (400 routes over 4
    experts: 128-row tiles) and with a larger count no route uses (64-row tiles); exact
    data, so both equal the oracle bit for bit."""
    from pegainfer_amd import _lib, ops
    from pegainfer_amd.ops import _ptr, _stream
    g = np.random.default_rng(bs + 7 * swiglu)
    E, N, K, T, topk = 4, 256, 512, 200, 2
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(np.ldexp(1.0, g.integers(-6, 1, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-4, 5, size=(T, K)).astype(np.float32))
    idx = g.integers(0, E, size=(T, topk)).astype(np.int32)
    w, packed = _setup(E, N, K, q, scale_bits)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    r = ops.moe_align_block_size(ws, dev(idx.reshape(-1)), T, T, 0)
    a = dev(a_bits)
    tw = dev(np.ones(T * topk, np.float32))
    width = N // 2 if swiglu else N
    outs = []
    for experts in (E, 16 * E):
        out = torch.full((T * topk, width), 7.0, dtype=torch.bfloat16, device="cuda")
        if swiglu:
            _lib.call("pega_wna16_w13_swiglu", _ptr(a), _ptr(out), None, 0,
                      _ptr(w.weight_packed_uint4b8), _ptr(w.weight_scale_permuted),
                      _ptr(r.sorted_token_ids), _ptr(r.expert_ids), _ptr(r.num_tokens_post_padded),
                      r.sorted_token_ids.numel(), bs, topk, T, N // 2, K, experts, 32, 0, _stream())
        else:
            _lib.call("pega_wna16_gemm", _ptr(a), _ptr(out), None, 0, _ptr(w.weight_packed_uint4b8),
                      _ptr(w.weight_scale_permuted), None, 0, _ptr(r.sorted_token_ids),
                      _ptr(r.expert_ids), _ptr(r.num_tokens_post_padded), _ptr(tw),
                      r.max_padded_tokens, bs, topk, False, T, N, K, experts, 32, 0, _stream())
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])
    routing = {k: host(v) for k, v in (("sorted_token_ids", r.sorted_token_ids),
                                       ("expert_ids", r.expert_ids),
                                       ("num_tokens_post_padded", r.num_tokens_post_padded))}
    ref = oracle.wna16_gemm(a_bits, packed, scale_bits, routing, np.ones((T, topk), np.float32),
                            moe_block_size=bs, top_k=topk, mul_topk_weights=False, size_m=T,
                            size_n=N, size_k=K, output=np.zeros((T * topk, N), np.uint16), threads=8)
    assert np.array_equal(outs[0], oracle.swiglu(ref, N // 2) if swiglu else ref)


@pytest.mark.parametrize("bs,K", [(8, 2080), (16, 1056)])
def test_gemm_decode_accepts_k_multiple_of_32(oracle, bs, K):
    """The reference accepts any K that is a multiple of 16 and of the group size 32
    (kimi_marlin_wna16.cu:284-286); the decode kernels work in 32-k groups, so an odd
    group count (K % 64 == 32) runs and matches the oracle bit for bit on exact data."""
    g = np.random.default_rng(K)
    E, N, T = 48, 128, 6
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(np.ldexp(1.0, g.integers(-4, 1, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-3, 4, size=(T, K)).astype(np.float32))
    idx = g.integers(0, 96, size=(T, 8))
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=8, bs=bs, mul=False, a_bits=a_bits, q=q,
                    scale_bits=scale_bits, idx=idx, tw=np.ones((T, 8), np.float32))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("K", [64, 96, 1056, 2080])
def test_decode16_uneven_and_empty_k_shares(oracle, K):
    """The 16x16x32 decode kernel (4 K-share waves per tile, picked when the launch has at
    least 4 workgroups per CU: here 77 m-blocks x 16 tiles = 1232 on 256 CUs) with group
    counts that 4 does not divide (33, 65: shares of 8 and 9, 16 and 17 groups) and with
    fewer groups than waves (2, 3: some waves add nothing), through the plain GEMM with the
    top-k weight and through W13 + SwiGLU (616 gate/up pairs: the paired launch, 4 waves
    per half).  Exact inputs, so both equal the oracle bit for bit."""
    from pegainfer_amd import ops
    E, T, topk, bs, inter = 48, 64, 8, 16, 512
    N = 2 * inter
    g = np.random.default_rng(4000 + K)
    q = g.integers(-8, 8, size=(E, N, K))
    scale_bits = oracle.f32_to_bf16(
        (2.0 ** g.integers(-6, -2, size=(E, N, K // 32))).astype(np.float32))
    a_bits = oracle.f32_to_bf16(g.integers(-2, 3, size=(T, K)).astype(np.float32))
    idx = np.stack([g.permutation(2 * E)[:topk] for _ in range(T)]).astype(np.int32)
    tw = oracle.bf16_to_f32(oracle.f32_to_bf16(g.random((T, topk)).astype(np.float32)))
    got, ref = _run(oracle, E=E, N=N, K=K, T=T, topk=topk, bs=bs, mul=True, a_bits=a_bits,
                    q=q, scale_bits=scale_bits, idx=idx, tw=tw, threads=16)
    assert np.array_equal(got, ref), f"GEMM K={K}"
    w, packed = _setup(E, N, K, q, scale_bits)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx.reshape(-1)), T, T, 0)
    assert ws.max_m_blocks * (N // 64) >= 4 * 256 and ws.max_m_blocks * (inter // 64) >= 2 * 256
    gws = ops.KimiMarlinWna16Workspace(ws.max_m_blocks, N, bs)
    act = torch.full((T * topk, inter), 3.0, dtype=torch.bfloat16, device="cuda")
    ops.wna16_w13_swiglu(gws, routing, dev(a_bits), w, act, top_k=topk, size_m=T)
    r = {k: host(v) for k, v in (("sorted_token_ids", routing.sorted_token_ids),
                                 ("expert_ids", routing.expert_ids),
                                 ("num_tokens_post_padded", routing.num_tokens_post_padded))}
    ref13 = oracle.wna16_gemm(a_bits, packed, scale_bits, r, np.ones((T, topk), np.float32),
                              moe_block_size=bs, top_k=topk, mul_topk_weights=False, size_m=T,
                              size_n=N, size_k=K, threads=16)
    local = idx.reshape(-1) < E
    got_act = host(act)
    assert np.array_equal(got_act[local], oracle.swiglu(ref13, inter)[local]), f"W13 K={K}"
    assert (got_act[~local] == 0x4040).all()
