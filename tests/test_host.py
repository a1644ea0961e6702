"""Host-side checks that need no GPU: the C-ABI library loads and exports every
symbol include/pega_moe.h declares, argument validation rejects bad shapes
before any launch (the reference's guards), and the Python mirror's shape
logic matches the reference's CPU unit tests
(pegainfer-kernels/src/ops/kimi_k2/experts.rs:1512-1641,
pegainfer-kimi-k2/src/runner/worker/runtime.rs:99-109)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "pega_moe.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(\w+)\(", text, flags=re.M)))


def test_header_declares_the_reference_entry_points():
    syms = _declared_symbols()
    for name in ["kimi_moe_marlin_align_block_size_cuda", "kimi_marlin_wna16_gemm_cuda",
                 "kimi_marlin_w13_swiglu_cuda", "kimi_marlin_w13_swiglu_expanded_cuda",
                 "kimi_marlin_sum_topk_rows_f32_cuda", "kimi_marlin_int4_reorder_weight_cuda",
                 "kimi_marlin_int4_reorder_scale_cuda", "kimi_marlin_int4_fuse_w13_cuda",
                 "kimi_residual_add_scaled_f32_cuda", "kimi_residual_add_scaled_bf16_cuda",
                 "kimi_add_f32_bf16_to_bf16_cuda", "kimi_deepep_build_marlin_routing_on_stream",
                 "kimi_k2_router_noaux_tc_cuda", "f32_to_bf16_cuda", "add_cuda", "gemm_cuda",
                 "gemm_graphsafe_cuda", "pegainfer_kernels_last_error"]:
        assert name in syms, name


def test_library_exports_every_declared_symbol():
    from pegainfer_amd import _lib
    L = _lib.lib()
    syms = _declared_symbols()
    assert len(syms) >= 20
    for name in syms:
        assert hasattr(L, name), f"{name} declared in pega_moe.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_hbm_probe_is_a_separate_library():
    """bench.py's streaming-read probe (measurement only) lives in its own library and
    rejects a misaligned or empty launch before touching the GPU; the expert-path
    library does not carry it."""
    from pegainfer_amd import _lib
    probe = ctypes.CDLL(os.path.join(ROOT, "pegainfer_amd", "libpega_hbm_probe.so"))
    fn = probe.pega_hbm_read_probe
    fn.argtypes = [ctypes.c_void_p, ctypes.c_ulonglong, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    assert fn(None, 1024, FAKE, 4, None) == 1
    assert fn(FAKE, 1000, FAKE, 4, None) == 1  # not a multiple of 16 bytes
    assert fn(FAKE, 1024, FAKE, 0, None) == 1
    assert not hasattr(_lib.lib(), "pega_hbm_read_probe")


def _call(name, *args):
    from pegainfer_amd import _lib
    return getattr(_lib.lib(), name)(*args), _lib.last_error()


NULL = None
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation rejects first


def test_align_rejects_reference_invalid_shapes():
    args = [FAKE] * 6
    # topk != 8 (kimi_experts.cu:217)
    rc, msg = _call("kimi_moe_marlin_align_block_size_cuda", *args, 7, 7, 96, 48, 8, 400, 50, NULL)
    assert rc == 1 and "topk" in msg
    # local_experts != 48
    rc, _ = _call("kimi_moe_marlin_align_block_size_cuda", *args, 7, 8, 96, 47, 8, 400, 50, NULL)
    assert rc == 1
    # block size 24 not allowed (:221)
    rc, msg = _call("kimi_moe_marlin_align_block_size_cuda", *args, 7, 8, 96, 48, 24, 400, 50, NULL)
    assert rc == 1 and "block_size" in msg
    # capacity below routes + E*(bs-1) = 56 + 336 = 392 (:224-229)
    rc, msg = _call("kimi_moe_marlin_align_block_size_cuda", *args, 7, 8, 96, 48, 8, 391, 49, NULL)
    assert rc == 1 and "capacity" in msg
    # null pointer
    rc, _ = _call("kimi_moe_marlin_align_block_size_cuda", NULL, *args[1:], 7, 8, 96, 48, 8, 392, 49, NULL)
    assert rc == 1
    # zero tokens
    rc, _ = _call("kimi_moe_marlin_align_block_size_cuda", *args, 0, 8, 96, 48, 8, 392, 49, NULL)
    assert rc == 1
    # the shape-general entry takes up to 512 local experts (one thread each)
    rc, msg = _call("pega_moe_align_block_size", *args, 7, 8, 0, 513, 8, 4000, 500, NULL)
    assert rc == 1 and "E=513" in msg


def test_gemm_rejects_reference_invalid_shapes():
    from pegainfer_amd import _lib
    f = _lib.lib().kimi_marlin_wna16_gemm_cuda

    def call(**kw):
        base = dict(workspace_len=4096, sorted_len=1232, bs=16, top_k=8, mul=False, m=64, n=4096,
                    k=7168, experts=48, group=32)
        base.update(kw)
        return f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, base["workspace_len"],
                 base["sorted_len"], base["bs"], base["top_k"], base["mul"], base["m"], base["n"],
                 base["k"], base["experts"], base["group"], 0, NULL)

    assert call(experts=47) == 1
    assert call(group=64) == 1
    assert call(bs=24) == 1
    assert call(n=4000) == 1
    assert call(k=7160) == 1
    assert call(m=0) == 1
    rc = f(FAKE, FAKE, NULL, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4096, 1232, 16, 8, False, 64,
           4096, 7168, 48, 32, 0, NULL)
    assert rc == 1  # c_tmp required (kimi_marlin_wna16.cu:272-274)
    odd = ctypes.c_void_p(0x1002)
    rc = f(FAKE, odd, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4096, 1232, 16, 8, False, 64,
           4096, 7168, 48, 32, 0, NULL)
    assert rc == 1  # the output rows are written with 16-byte stores


def test_gemm_rejects_a_lock_workspace_below_the_reference_floor():
    """kimi_marlin_wna16.cu:305-309: workspace_len < min(n_tiles * (sorted_len / bs),
    4 * sm_count) is INVALID_VALUE, although the locks themselves are not used here."""
    from pegainfer_amd import _lib
    f = _lib.lib().kimi_marlin_wna16_gemm_cuda

    def call(workspace_len, sm_count, sorted_len=1232, bs=16, n=4096):
        rc = f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, workspace_len,
               sorted_len, bs, 8, False, 64, n, 7168, 48, 32, sm_count, NULL)
        return rc, _lib.last_error()
    # 64 column tiles x 77 m-blocks = 4928 > 4 * 256 = 1024: the floor is 1024
    rc, msg = call(1023, 256)
    assert rc == 1 and "workspace_len" in msg
    # 4 * 78 = 312 with the reference's H20 SM count
    rc, msg = call(311, 78)
    assert rc == 1 and "workspace_len" in msg
    # a tiny problem: 1 m-block x 1 column tile = 1 lock
    rc, msg = call(0, 256, sorted_len=16, n=64)
    assert rc == 1 and "workspace_len" in msg
    # at the floor the check passes (the call then fails only for want of a device)
    rc, msg = call(1024, 256)
    assert "workspace_len" not in msg
    # K % 16 == 0 but K % 32 != 0: the group size does not divide K
    rc = f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4096, 1232, 16, 8, False,
           64, 4096, 7168 + 16, 48, 32, 256, NULL)
    assert rc == 1


def test_deepep_routing_rejects_more_than_64_experts_like_the_reference():
    """kimi_experts.cu:446: num_local_experts > kRoutingBuilderMaxExperts (64) -> 1."""
    rc, msg = _call("kimi_deepep_build_marlin_routing_on_stream", FAKE, FAKE, FAKE, FAKE, 65, 8,
                    8, 1000, 125, NULL)
    assert rc == 1 and "64" in msg


def test_router_noaux_tc_rejects_like_the_reference():
    """kimi_router.cu:162-171: null pointers, token counts, n_experts != 384, topk != 8,
    route_scale <= 0 -> INVALID_VALUE; the MFMA logits GEMM needs hidden_dim % 32 == 0
    (801 otherwise)."""
    def call(active=64, padded=64, hidden=7168, experts=384, topk=8, scale=1.0, ptrs=None):
        p = ptrs if ptrs is not None else [FAKE] * 6
        return _call("kimi_k2_router_noaux_tc_cuda", *p, active, padded, hidden, experts, topk,
                     ctypes.c_float(scale), NULL)
    assert call(experts=256)[0] == 1
    assert call(topk=6)[0] == 1
    assert call(active=65)[0] == 1          # active_tokens > padded_tokens
    assert call(active=0)[0] == 1
    assert call(padded=0, active=0)[0] == 1
    assert call(hidden=0)[0] == 1
    assert call(scale=0.0)[0] == 1
    assert call(scale=float("nan"))[0] == 1
    assert call(ptrs=[FAKE] * 5 + [NULL])[0] == 1
    rc, msg = call(hidden=7168 + 16)
    assert rc == 801 and "K" in msg
    # the MFMA logits GEMM reads hidden and gate_weight with 16-byte loads: a misaligned
    # buffer is a layout this build does not support (801), as the header states
    odd = ctypes.c_void_p(0x1008)
    rc, msg = call(ptrs=[odd] + [FAKE] * 5)
    assert rc == 801 and "aligned" in msg
    rc, msg = call(ptrs=[FAKE, odd] + [FAKE] * 4)
    assert rc == 801 and "aligned" in msg
    for name in ("gemm_cuda", "gemm_graphsafe_cuda"):
        rc, msg = _call(name, FAKE, odd, FAKE, 4096, 64, 7168, NULL)
        assert rc == 801 and "aligned" in msg
    rc, msg = _call("pega_dense_w13_swiglu", odd, FAKE, FAKE, 2048, 64, 7168, NULL)
    assert rc == 801 and "aligned" in msg


def test_dense_gemm_w_size_is_not_limited_only_its_workgroup_span():
    """A W larger than 2 GiB (the unsharded Kimi lm_head, 163840 x 7168 bf16) passes the
    range checks: each workgroup addresses only its own 32 rows.  With the SwiGLU
    epilogue a workgroup spans gate to up rows, so (I + 16) * K * 2 must stay below 2 GiB."""
    rc, msg = _call("gemm_cuda", FAKE, FAKE, FAKE, 163840, 64, 7168, NULL)
    assert "2 GiB" not in msg  # (on a host without a GPU it then fails for want of a device)
    rc, msg = _call("gemm_graphsafe_cuda", FAKE, FAKE, FAKE, 163840, 64, 7168, NULL)
    assert "2 GiB" not in msg
    rc, msg = _call("pega_dense_w13_swiglu", FAKE, FAKE, FAKE, 150000, 64, 7168, NULL)
    assert rc == 801 and "2 GiB" in msg
    rc, msg = _call("gemm_cuda", FAKE, FAKE, FAKE, 4096, 200_000, 7168, NULL)  # X 2.87 GB
    assert rc == 801 and "2 GiB" in msg


def test_elementwise_reference_symbols_reject_bad_arguments():
    assert _call("f32_to_bf16_cuda", NULL, FAKE, 8, NULL)[0] == 1
    assert _call("f32_to_bf16_cuda", FAKE, FAKE, -1, NULL)[0] == 1
    assert _call("f32_to_bf16_cuda", FAKE, FAKE, 0, NULL)[0] == 0
    assert _call("add_cuda", FAKE, NULL, FAKE, 8, NULL)[0] == 1
    assert _call("add_cuda", FAKE, FAKE, FAKE, 0, NULL)[0] == 0
    assert _call("pega_moe_join_routed_shared_bf16", FAKE, FAKE, NULL, 8, NULL)[0] == 1
    assert _call("pega_moe_join_routed_shared_bf16", FAKE, FAKE, FAKE, 0, NULL)[0] == 0


def test_repack_reference_symbols_return_invalid_value_on_every_failure():
    """kimi_marlin_int4.cu:190,220,254,262 map every failure (a launch failure included) to
    CUDA_ERROR_INVALID_VALUE; shape failures are 1 as well."""
    assert _call("kimi_marlin_int4_reorder_weight_cuda", FAKE, FAKE, 7168, 2048, 48, 16,
                 NULL)[0] == 1
    assert _call("kimi_marlin_int4_reorder_scale_cuda", NULL, FAKE, 7168, 2048, 48, 32,
                 NULL)[0] == 1


def test_gemm_entries_reject_shapes_past_the_32_bit_ranges():
    """One expert's weights are addressed through a 32-bit range (<= 4 GiB) and the
    activations through one of at most 2 GiB (offset 2^31 reads zeros for rows that
    are not routed here); larger shapes are refused before any launch."""
    def gemm(m, n, k):
        return _call("pega_wna16_gemm", FAKE, FAKE, FAKE, ctypes.c_longlong(0), FAKE, FAKE, FAKE,
                     0, FAKE, FAKE, FAKE, FAKE, 4096, 64, 1, False, m, n, k, 1, 32, 256, NULL)
    rc, reason = gemm(200_000, 4096, 7168)       # input 2.87 GB
    assert rc == 801 and "2 GiB" in reason
    assert gemm(1, 65536, 131072)[0] == 801      # 4.29 GB of weights per expert
    rc = _call("pega_wna16_w13_swiglu", FAKE, FAKE, NULL, ctypes.c_longlong(0), FAKE, FAKE, FAKE,
               FAKE, FAKE, 4096, 64, 1, 200_000, 2048, 7168, 1, 32, 256, NULL)[0]
    assert rc == 801
    assert _call("pega_wna16_prefill_pair", ctypes.byref(_problem()),
                 ctypes.byref(_problem(size_m=200_000, size_k=7168)), NULL)[0] == 801


def test_repack_and_elementwise_reject_bad_arguments():
    assert _call("kimi_marlin_int4_reorder_weight_cuda", FAKE, FAKE, 64, 64, 47, 32, NULL)[0] == 1
    assert _call("kimi_marlin_int4_reorder_weight_cuda", FAKE, FAKE, 64, 60, 48, 32, NULL)[0] == 1
    assert _call("kimi_marlin_int4_reorder_scale_cuda", FAKE, FAKE, 64, 64, 48, 16, NULL)[0] == 1
    assert _call("kimi_marlin_int4_fuse_w13_cuda", *([FAKE] * 5), NULL, 64, 64, 48, 32, NULL)[0] == 1
    assert _call("kimi_marlin_w13_swiglu_cuda", FAKE, FAKE, -1, 64, NULL)[0] == 1
    assert _call("kimi_marlin_w13_swiglu_cuda", FAKE, FAKE, 0, 64, NULL)[0] == 0  # no-op
    assert _call("kimi_marlin_sum_topk_rows_f32_cuda", FAKE, FAKE, 4, 0, 64, NULL)[0] == 1
    assert _call("kimi_marlin_sum_topk_rows_f32_cuda", FAKE, FAKE, 0, 8, 64, NULL)[0] == 0
    assert _call("kimi_residual_add_scaled_f32_cuda", FAKE, FAKE, NULL, ctypes.c_float(2.8), FAKE,
                 8, NULL)[0] == 1
    assert _call("kimi_add_f32_bf16_to_bf16_cuda", FAKE, FAKE, FAKE, -1, NULL)[0] == 1
    assert _call("pega_kimi_router_select", FAKE, FAKE, FAKE, FAKE, 4, 384, 400,
                 ctypes.c_float(1.0), NULL)[0] == 1
    assert _call("pega_dsv2_router_select", FAKE, FAKE, FAKE, 4, 64, 0, NULL)[0] == 1
    # local-route combine: hidden % 8 and experts > 0 required
    assert _call("pega_moe_combine_local_f32", FAKE, FAKE, NULL, FAKE, 4, 8, 100, 0, 48,
                 NULL)[0] == 1
    assert _call("pega_moe_combine_local_f32", FAKE, FAKE, NULL, FAKE, 4, 8, 7168, 0, 0,
                 NULL)[0] == 1
    # one workgroup per (token, 1024-column chunk): the grid must fit 2^31 - 1
    assert _call("pega_moe_combine_local_f32", FAKE, FAKE, NULL, FAKE, 400_000_000, 8, 7168, 0,
                 48, NULL)[0] == 1


def test_fused_w13_swiglu_rejects_bad_arguments():
    def call(**kw):
        base = dict(partials_len=1 << 20, sorted_len=15, bs=8, top_k=1, m=1, inter=2048, k=7168,
                    experts=1, group=32, partials=FAKE)
        base.update(kw)
        return _call("pega_wna16_w13_swiglu", FAKE, FAKE, base["partials"],
                     ctypes.c_longlong(base["partials_len"]), FAKE, FAKE, FAKE, FAKE, FAKE,
                     base["sorted_len"], base["bs"], base["top_k"], base["m"], base["inter"],
                     base["k"], base["experts"], base["group"], 0, NULL)
    assert call(bs=24)[0] == 1             # block sizes 8, 16, 32, 48, 64 only
    assert call(group=64)[0] == 1
    assert call(inter=2000)[0] == 1        # width must be a multiple of 64
    assert call(k=7160)[0] == 1            # K must be a multiple of the group (32)
    assert call(k=7168 + 32, bs=64)[0] == 801  # the prefill tile kernel stages 64 k at a time
    assert call(m=0)[0] == 1
    odd = ctypes.c_void_p(0x1008)
    rc = _call("pega_wna16_w13_swiglu", FAKE, odd, FAKE, ctypes.c_longlong(1 << 20), FAKE, FAKE,
               FAKE, FAKE, FAKE, 15, 8, 1, 1, 2048, 7168, 1, 32, 0, NULL)[0]
    assert rc == 1                         # act is written with 16-byte stores


def _problem(**kw):
    from pegainfer_amd import _lib
    f = dict(input=0x1000, output=0x1000, act=None, b_qweight=0x1000, b_scales=0x1000,
             sorted_token_ids=0x1000, expert_ids=0x1000, num_tokens_post_padded=0x1000,
             topk_weights=0x1000, sorted_token_ids_len=640, moe_block_size=64, top_k=1,
             mul_topk_weights=0, size_m=512, size_n=2048, size_k=1408, local_experts=1,
             group_size=32)
    f.update(kw)
    return _lib.Wna16Problem(**f)


def test_prefill_pair_rejects_bad_arguments():
    def call(a, b):
        return _call("pega_wna16_prefill_pair", ctypes.byref(a) if a is not None else None,
                     ctypes.byref(b) if b is not None else None, NULL)
    ok = _problem()
    assert call(None, ok)[0] == 1
    assert call(ok, None)[0] == 1
    assert call(ok, _problem(moe_block_size=16))[0] == 801   # decode sizes: other kernels
    assert call(_problem(moe_block_size=24), ok)[0] == 801
    assert call(ok, _problem(input=0x1008))[0] == 1           # 16-byte aligned input
    assert call(ok, _problem(act=0x1000, mul_topk_weights=1))[0] == 1  # no weight with SwiGLU
    assert call(ok, _problem(act=0x1000, size_n=2048 + 64))[0] == 801  # gate/up 64-col tiles
    assert call(ok, _problem(output=None))[0] == 1
    assert call(ok, _problem(mul_topk_weights=1, topk_weights=None))[0] == 1
    assert call(ok, _problem(group_size=64))[0] == 1
    rc, reason = call(ok, _problem(size_k=1400))
    assert rc == 801 and "second" in reason


def test_problem_struct_matches_the_header(tmp_path):
    """The ctypes mirror of pega_wna16_problem has the C layout: gcc compiles the
    header and prints sizeof and every offsetof."""
    import shutil
    import subprocess
    from pegainfer_amd import _lib
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    names = [f[0] for f in _lib.Wna16Problem._fields_]
    src = tmp_path / "layout.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"pega_moe.h\"\n"
                   "int main(void) {\n  printf(\"%zu\\n\", sizeof(pega_wna16_problem));\n" +
                   "".join(f"  printf(\"%zu\\n\", offsetof(pega_wna16_problem, {n}));\n"
                           for n in names) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.Wna16Problem) == 112
    assert got[1:] == [getattr(_lib.Wna16Problem, n).offset for n in names]


# ------------------------------------------------------------- Python mirror logic
def test_manifest_shapes_match_reference_unit_tests():
    from pegainfer_amd import ops
    m = ops.KimiInt4WeightManifest.ep8(ops.KimiInt4ExpertRole.W1Gate, 3,
                                        ops.KimiInt4NibbleOrder.LowThenHigh)
    m.validate()
    assert m.local_experts == 48 and m.local_expert_offset == 144
    assert m.packed_shape.elements() == 48 * 2048 * (7168 // 2)
    assert m.scale_shape.elements() == 48 * 2048 * (7168 // 32)
    d = ops.KimiInt4WeightManifest.ep8(ops.KimiInt4ExpertRole.W2Down, 0,
                                        ops.KimiInt4NibbleOrder.LowThenHigh)
    d.validate()
    assert d.logical_shape == ops.KimiInt4LogicalShape(out_dim=7168, in_dim=2048)
    assert d.packed_shape.elements() == 48 * 7168 * (2048 // 2)
    assert d.marlin_packed_u32_elements() * 4 == d.packed_shape.elements()
    import dataclasses
    bad = dataclasses.replace(m, group_size=64)
    with pytest.raises(ValueError):
        bad.validate()
    with pytest.raises(ValueError):
        dataclasses.replace(m, local_experts=47).validate()


def test_capacity_and_block_size_policy():
    from pegainfer_amd import ops
    cap = ops.marlin_padded_route_capacity(7, 8)
    assert cap == 7 * 8 + 48 * 7 and -(-cap // 8) == 49
    # runtime.rs:99-109: smallest bs with T*8/48/bs < 0.9
    # (T < 5.4 * bs): 8 up to 43 tokens, 16 up to 86, 32 up to 172, 48 up to 259
    for t, bs in [(1, 8), (43, 8), (44, 16), (64, 16), (86, 16), (87, 32), (172, 32),
                  (173, 48), (259, 48), (260, 64), (4096, 64)]:
        assert ops.kimi_marlin_block_size(t) == bs, t
    with pytest.raises(ValueError):
        ops.validate_marlin_block_size(24)


def test_synth_routing_generators_are_seeded_and_shaped():
    import numpy as np
    from pegainfer_amd import synth
    idx, w = synth.zipf_local_topk(synth.rng(5, 1), 512, routes_target=800)
    idx2, _ = synth.zipf_local_topk(synth.rng(5, 1), 512, routes_target=800)
    assert np.array_equal(idx, idx2)
    assert idx.shape == (512, 8) and np.allclose(w.sum(1), 1.0, atol=1e-6)
    for row in idx:
        assert len(set(row.tolist())) == 8
        assert 1 <= (row < 48).sum() <= 2
    counts = np.bincount(idx[idx < 48], minlength=48)
    assert counts.max() > 4 * max(1, np.median(counts))  # skewed


def test_router_wrappers_reject_short_inputs_before_the_device():
    """The select kernels read active_tokens rows of logits and n_experts biases on the
    device: the host wrappers reject tensors that do not cover them (no launch)."""
    import torch
    from pegainfer_amd import ops
    f32, i32 = torch.float32, torch.int32
    ws = ops.KimiMarlinRouteWorkspace(4, 16, topk=8, local_experts=48, device="cpu")
    ok = dict(logits=torch.zeros(4, 384, dtype=f32), bias=torch.zeros(384, dtype=f32),
              topk_weight=torch.zeros(32, dtype=f32), topk_idx=torch.zeros(32, dtype=i32))

    def route_align(**kw):
        a = dict(ok, **kw)
        ops.kimi_route_align(ws, a["logits"], a["bias"], a["topk_weight"], a["topk_idx"], 4, 0)

    def select(**kw):
        a = dict(ok, **kw)
        ops.kimi_router_select(a["logits"], a["bias"], a["topk_weight"], a["topk_idx"], 4)

    for fn in (route_align, select):
        with pytest.raises(Exception, match="logits must cover"):
            fn(logits=torch.zeros(3, 384, dtype=f32))
        with pytest.raises(Exception, match="bias must cover"):
            fn(bias=torch.zeros(383, dtype=f32))
        with pytest.raises(Exception, match="topk_idx"):
            fn(topk_idx=torch.zeros(31, dtype=i32))
    with pytest.raises(Exception, match="logits must cover"):
        ops.dsv2_router_select(torch.zeros(7, 64, dtype=f32), torch.zeros(48, dtype=f32),
                               torch.zeros(48, dtype=i32), 8, 6)
