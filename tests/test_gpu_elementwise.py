"""GPU parity of the elementwise stages (K3 SwiGLU, K3' expanded SwiGLU, K4
top-k sum, K8 residual joins, K10 add, DeepSeek-V2-Lite weighted combine):
bit-exact with the oracle, which restates the reference's rounding points."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def _bf16_rand(g, shape, scale=1.0):
    from oracle import oracle
    return oracle.f32_to_bf16((g.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("rows,inter", [(1, 2048), (512, 2048), (37, 1408), (5, 100)])
def test_swiglu_bit_exact(oracle, rows, inter):
    from pegainfer_amd import ops
    g = np.random.default_rng(rows + inter)
    w13 = _bf16_rand(g, (rows, 2 * inter), 3.0)
    w13[0, :3] = [0, 0x8000, 0x7F80]  # +0, -0, +inf gate
    out = torch.zeros(rows, inter, dtype=torch.bfloat16, device="cuda")
    ops.kimi_marlin_w13_swiglu(dev(w13), out, rows, inter)
    ref = oracle.swiglu(w13, inter)
    got = host(out)
    fin = np.isfinite((ref.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(got[fin], ref[fin])


def test_swiglu_every_bf16_gate(oracle):
    """Every bf16 gate value (all 65536 bit patterns), once with up = 1 (the result is
    then bf16(silu) itself) and once with random up values, against the checker's
    SwiGLU with the exact exponential: the kernels' fast exponential path, taken when
    the fast silu is clear of a bf16 rounding midpoint, must give the same bits for
    every gate they can be passed."""
    from pegainfer_amd import ops
    inter = 65536
    gates = np.arange(inter, dtype=np.uint32).astype(np.uint16)
    w13 = np.empty((2, 2 * inter), np.uint16)
    w13[:, :inter] = gates
    w13[0, inter:] = 0x3F80  # up = 1.0
    w13[1, inter:] = _bf16_rand(np.random.default_rng(11), (inter,), 2.0)
    out = torch.zeros(2, inter, dtype=torch.bfloat16, device="cuda")
    ops.kimi_marlin_w13_swiglu(dev(w13), out, 2, inter)
    got, ref = host(out), oracle.swiglu(w13, inter)
    as_f32 = lambda b: (b.astype(np.uint32) << 16).view(np.float32)
    nan_ref = np.isnan(as_f32(ref))
    assert np.array_equal(np.isnan(as_f32(got)), nan_ref)
    assert np.array_equal(got[~nan_ref], ref[~nan_ref])


def test_swiglu_expanded_reads_rows_on_device(oracle):
    from pegainfer_amd import ops
    g = np.random.default_rng(9)
    max_rows, inter = 300, 2048
    w13 = _bf16_rand(g, (max_rows, 2 * inter))
    for live in (0, 17, 300, 1000):  # 1000 is clamped to max_rows
        out = torch.full((max_rows, inter), 3.0, dtype=torch.bfloat16, device="cuda")
        ops.kimi_marlin_w13_swiglu_expanded(dev(w13), dev(np.array([live], np.int32)), out,
                                            max_rows, inter)
        got = host(out)
        n = min(live, max_rows)
        if n:
            assert np.array_equal(got[:n], oracle.swiglu(w13[:n], inter))
        assert (got[n:] == 0x4040).all()  # untouched rows keep bf16(3.0)


@pytest.mark.parametrize("T,topk,H", [(1, 8, 7168), (64, 8, 7168), (3, 6, 2048), (2, 8, 100)])
def test_sum_topk_rows_bit_exact(oracle, T, topk, H):
    from pegainfer_amd import ops
    g = np.random.default_rng(T * H)
    r = _bf16_rand(g, (T * topk, H), 50.0)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    ops.kimi_marlin_sum_topk_rows_f32(dev(r), T, out, topk, H)
    assert np.array_equal(host(out), oracle.sum_topk_rows(r, T, topk, H))


def test_weighted_topk_sum_bit_exact(oracle):
    from pegainfer_amd import ops
    g = np.random.default_rng(2)
    T, topk, H = 512, 6, 2048
    r = _bf16_rand(g, (T * topk, H))
    w = g.random((T, topk)).astype(np.float32)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    ops.weighted_topk_sum_f32(dev(r), dev(w), T, out, topk, H)
    assert np.array_equal(host(out), oracle.weighted_topk_sum(r, w, T, topk, H))


@pytest.mark.parametrize("T,topk,H,gs,E,weighted", [(64, 8, 7168, 0, 48, False),
                                                     (5, 8, 7168, 96, 48, False),
                                                     (512, 6, 2048, 0, 64, True),
                                                     (33, 6, 2048, 16, 20, True),
                                                     (40, 5, 7168, 8, 30, True),
                                                     (7, 3, 1032, 0, 10, False)])
def test_combine_local_equals_zero_filled_combine(oracle, T, topk, H, gs, E, weighted):
    """pega_moe_combine_local_f32 never reads rows of non-local routes (they hold
    NaN here) and equals the zero-filled full combine bit for bit.  Top-k 8 and 6
    take the compile-time paths, 5 and 3 the runtime one; 1032 columns end in a
    partial 1024-column chunk."""
    from pegainfer_amd import ops
    g = np.random.default_rng(T + topk + gs)
    idx = g.integers(0, 384 if E == 48 else 64, size=(T, topk)).astype(np.int32)
    local = ((idx - gs) >= 0) & ((idx - gs) < E)
    r = _bf16_rand(g, (T * topk, H), 50.0)
    r_garbage = r.copy()
    r_garbage[~local.reshape(-1)] = 0x7FC0  # bf16 NaN: any read would show
    r_zero = r.copy()
    r_zero[~local.reshape(-1)] = 0
    w = g.random((T, topk)).astype(np.float32)
    out = torch.full((T, H), 7.0, dtype=torch.float32, device="cuda")
    ops.moe_combine_local_f32(dev(r_garbage), dev(idx), dev(w) if weighted else None, T, out,
                              topk, H, gs, E)
    ref = (oracle.weighted_topk_sum(r_zero, w, T, topk, H) if weighted
           else oracle.sum_topk_rows(r_zero, T, topk, H))
    got = host(out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # the same combine with the DSV2 join in one launch: the two-rounding join of ref
    sh = _bf16_rand(g, (T, H), 4.0)
    joined = torch.full((T, H), 5.0, dtype=torch.bfloat16, device="cuda")
    ops.moe_combine_join(dev(r_garbage), dev(idx), dev(w) if weighted else None, dev(sh), joined,
                         T, topk, H, gs, E)
    want = oracle.dsv2_join(ref.reshape(-1), sh.reshape(-1)).reshape(T, H)
    assert np.array_equal(host(joined), want)


def test_residual_joins_bit_exact(oracle):
    from pegainfer_amd import ops
    g = np.random.default_rng(3)
    n = 64 * 7168
    h, p = _bf16_rand(g, n), _bf16_rand(g, n)
    rf = g.standard_normal(n).astype(np.float32)
    rb = _bf16_rand(g, n)
    out = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
    ops.kimi_residual_add_scaled_f32(dev(h), dev(p), dev(rf), 2.827, out)
    assert np.array_equal(host(out), oracle.residual_add_scaled_f32(h, p, rf, 2.827))
    ops.kimi_residual_add_scaled_bf16(dev(h), dev(p), dev(rb), 2.827, out)
    assert np.array_equal(host(out), oracle.residual_add_scaled_bf16(h, p, rb, 2.827))
    ops.kimi_add_f32_bf16_to_bf16(dev(rf), dev(h), out)
    assert np.array_equal(host(out), oracle.add_f32_bf16(rf, h))


def test_f32_to_bf16_add_and_dsv2_join_bit_exact(oracle):
    """f32_to_bf16_cuda and add_cuda (the reference symbols) and the fused DeepSeek-V2-Lite
    join pega_moe_join_routed_shared_bf16, against the oracle's two-rounding join; the
    planted pairs are ones where a single rounding of routed + shared differs."""
    from pegainfer_amd import ops
    g = np.random.default_rng(31)
    for n in (512 * 2048, 1000, 7):  # vector path, then element tails / scalar path
        r = (g.standard_normal(n) * 3).astype(np.float32)
        r[:2] = [1.0 + 2 ** -8 + 2 ** -12, 1.0 + 2 ** -9]
        sh = _bf16_rand(g, n)
        sh[:2] = oracle.f32_to_bf16(np.array([2 ** -8, 2 ** -9], np.float32))
        rb = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
        ops.f32_to_bf16(dev(r), rb)
        assert np.array_equal(host(rb), oracle.f32_to_bf16_n(r))
        out = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
        ops.add_bf16(rb, dev(sh), out)
        want = oracle.dsv2_join(r, sh)
        assert np.array_equal(host(out), want)
        fused = torch.full((n,), 5.0, dtype=torch.bfloat16, device="cuda")
        ops.moe_join_routed_shared(dev(r), dev(sh), fused)
        assert np.array_equal(host(fused), want)
        assert want[0] != oracle.add_f32_bf16(r[:1], sh[:1])[0]
