"""GPU parity of pega_wna16_w13_swiglu_noalloc, the entry point that allocates nothing
(the K-split partials live in the library's static per-device scratch), against
pega_wna16_w13_swiglu given a caller workspace: bit for bit, on two calls in a row (the
second with a smaller input), a no-split shape, a split the scratch cannot hold (run
unsplit, as the workspace entry does with a workspace of the scratch's size), and a first
call made inside a HIP graph capture (the scratch address is looked up there), replayed.
The capture test comes first in this file, so in a fresh process its call is the first."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import dev, host

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 1 << 19  # the static scratch: 2 MiB per device


def _problem(E, T, topk, bs, inter, K, seed):
    from pegainfer_amd import layer, ops, synth
    g = synth.rng(90 + seed, 1)
    gate, up = synth.int4_checkpoint(g, E, inter, K), synth.int4_checkpoint(g, E, inter, K)
    w13 = layer.package_w13(gate, up)
    x = dev(synth.normal_bf16(g, (T, K)))
    idx = np.random.default_rng(seed).integers(0, E, size=(T, topk)).astype(np.int32)
    ws = ops.KimiMarlinRouteWorkspace(T, bs, topk=topk, local_experts=E)
    routing = ops.moe_align_block_size(ws, dev(idx), T, T, 0)
    return w13, x, routing


def _call(name, routing, x, w13, act, T, topk, inter, K, E, partials=None):
    from pegainfer_amd import _lib
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    s = torch.cuda.current_stream().cuda_stream
    common = (p(routing.sorted_token_ids), p(routing.expert_ids),
              p(routing.num_tokens_post_padded), routing.sorted_token_ids.numel(),
              routing.block_size, topk, T, inter, K, E, 32, 0, s)
    L = _lib.lib()
    if name == "noalloc":
        return L.pega_wna16_w13_swiglu_noalloc(p(x), p(act), p(w13.weight_packed_uint4b8),
                                               p(w13.weight_scale_permuted), *common)
    return L.pega_wna16_w13_swiglu(p(x), p(act), p(partials),
                                   ctypes.c_longlong(partials.numel()),
                                   p(w13.weight_packed_uint4b8), p(w13.weight_scale_permuted),
                                   *common)


def test_noalloc_first_call_inside_graph_capture_then_replays():
    """The first call on the device (and so hipGetSymbolAddress) happens while the stream
    is being captured; two replays, with eager work and synchronisation between them, equal
    the workspace entry bit for bit."""
    E, T, topk, bs, inter, K = 1, 8, 1, 8, 2048, 7168
    w13, x, routing = _problem(E, T, topk, bs, inter, K, 5)
    routes = T * topk
    partials = torch.zeros(SCRATCH_FLOATS, dtype=torch.float32, device="cuda")
    ref = torch.full((routes, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert _call("workspace", routing, x, w13, ref, T, topk, inter, K, E, partials) == 0
    got = torch.full((routes, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g):
        rcs.append(_call("noalloc", routing, x, w13, got, T, topk, inter, K, E))
    assert rcs == [0]
    r = host(ref)
    for _ in range(2):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(got), r)


def _run_pair(E, T, topk, bs, inter, K, seed):
    """Both entries on the same problem, the workspace entry with a workspace of the
    static scratch's size: the documented equality (the share count depends on the
    buffer's size)."""
    w13, x, routing = _problem(E, T, topk, bs, inter, K, seed)
    routes = T * topk
    partials = torch.zeros(SCRATCH_FLOATS, dtype=torch.float32, device="cuda")
    ref = torch.full((routes, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    got = torch.full((routes, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert _call("workspace", routing, x, w13, ref, T, topk, inter, K, E, partials) == 0
    assert _call("noalloc", routing, x, w13, got, T, topk, inter, K, E) == 0
    torch.cuda.synchronize()
    routed = host(routing.sorted_token_ids)
    rows = np.unique(routed[routed < routes])
    r, g_ = host(ref), host(got)
    assert np.array_equal(g_[rows], r[rows])
    return rows.size


def test_noalloc_matches_workspace_entry_twice_second_smaller():
    # one Kimi expert at batch 8, then batch 2: the split path (partials in the scratch)
    n1 = _run_pair(E=1, T=8, topk=1, bs=8, inter=2048, K=7168, seed=1)
    n2 = _run_pair(E=1, T=2, topk=1, bs=8, inter=2048, K=7168, seed=2)
    assert n1 == 8 and n2 == 2


def test_noalloc_no_split_shape_and_scratch_limit():
    # C3-like: 77 capacity blocks x 8 column tiles, two workgroups per CU: no split
    _run_pair(E=48, T=64, topk=8, bs=16, inter=256, K=1024, seed=3)
    # a split is wanted (14 capacity blocks x 32 tiles < 2 workgroups per CU) but two shares
    # of 200 routes x 2048 columns exceed the 524,288-float scratch: it runs unsplit, as the
    # workspace entry does with a workspace of the scratch's size
    n = _run_pair(E=1, T=200, topk=1, bs=16, inter=1024, K=1024, seed=4)
    assert n == 200
