"""A routed-expert decode layer (router select + permutation + W13 + SwiGLU +
W2 + local combine) captured into a HIP graph and replayed: every replay,
with eager launches and host synchronisation between replays, must give the
eager result bit for bit (the captured launches hold no memset nodes)."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    from pegainfer_amd import layer, ops, synth
    E, H, I, T = 48, 512, 256, 16
    g = synth.rng(9, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    moe = layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                              max_tokens=T, topk=8, block_size=ops.kimi_marlin_block_size(T))
    hidden = dev(synth.normal_bf16(synth.rng(9, 2), (T, H)).view(np.int16)).view(torch.bfloat16)
    logits_a = dev(synth.rng(9, 3).standard_normal((T, 384), dtype=np.float32))
    logits_b = dev(synth.rng(9, 4).standard_normal((T, 384), dtype=np.float32))
    logits = torch.empty_like(logits_a)
    bias = torch.zeros(384, dtype=torch.float32, device="cuda")
    tw = torch.zeros(T, 8, dtype=torch.float32, device="cuda")
    ti = torch.zeros(T, 8, dtype=torch.int32, device="cuda")
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")

    def step():
        ops.kimi_router_select(logits, bias, tw, ti, T)
        moe.forward(hidden, ti, tw, out)

    refs = {}
    for name, src in (("a", logits_a), ("b", logits_b)):
        logits.copy_(src)
        step()
        torch.cuda.synchronize()
        refs[name] = host(out).copy()
    assert not np.array_equal(refs["a"], refs["b"])  # the two routings differ

    logits.copy_(logits_a)
    graph = layer.capture_graph(step)
    for i in range(4):
        name = "ab"[i % 2]
        logits.copy_(logits_a if name == "a" else logits_b)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint32), refs[name].view(np.uint32)), (i, name)
        # eager work between replays reuses the same buffers
        step()
        torch.cuda.synchronize()
        assert np.array_equal(host(out).view(np.uint32), refs[name].view(np.uint32))


def test_full_decode_layer_graph_replays_match_eager():
    """The Kimi decode layer with its shared expert (dense bf16 GEMMs) and the
    residual join, captured once: replays under two routings, with eager runs of
    the same layer between them, give the eager bits every time."""
    from pegainfer_amd import layer, ops, synth
    E, H, I, T, SI = 48, 512, 256, 16, 512
    g = synth.rng(10, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    routed = layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                                 max_tokens=T, topk=8, block_size=ops.kimi_marlin_block_size(T))
    bf = lambda a: dev(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)  # noqa: E731
    gu = bf(synth.normal_bf16(g, (2 * SI, H), std=0.03))
    dn = bf(synth.normal_bf16(g, (H, SI), std=0.03))
    moe = layer.KimiMoeDecodeLayer(routed, layer.KimiSharedExpert(gu, dn, max_tokens=T))
    hidden = bf(synth.normal_bf16(g, (T, H)))
    normed = bf(synth.normal_bf16(g, (T, H)))
    logits_a = dev(g.standard_normal((T, 384), dtype=np.float32))
    logits_b = dev(g.standard_normal((T, 384), dtype=np.float32))
    logits = torch.empty_like(logits_a)
    bias = torch.zeros(384, dtype=torch.float32, device="cuda")
    out = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")

    def step():
        moe.forward(hidden, normed, logits, bias, out)

    refs = {}
    for name, src in (("a", logits_a), ("b", logits_b)):
        logits.copy_(src)
        step()
        torch.cuda.synchronize()
        refs[name] = host(out).copy()
    assert not np.array_equal(refs["a"], refs["b"])

    logits.copy_(logits_a)
    graph = layer.capture_graph(step)
    for i in range(4):
        name = "ab"[i % 2]
        logits.copy_(logits_a if name == "a" else logits_b)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), refs[name]), (i, name)
        step()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), refs[name])
