/*
 * pega_moe.h -- C ABI of libpega_moe_hip.so, the MI355X (gfx950) quantized
 * MoE expert path (W4A16: INT4 group-32 symmetric weights, bf16 activations,
 * fp32 accumulation).
 *
 * Conventions (as in the reference's FFI, pegainfer-kernels/src/ffi/kimi.rs
 * and src/ffi.rs:5):
 *   - bf16 tensors are passed as uint16_t bit patterns;
 *   - all pointers are device pointers, caller-owned; no entry point
 *     allocates, synchronises or copies to the host;
 *   - `stream` is a hipStream_t (the reference passes a CUstream);
 *   - return value: 0 success, 1 invalid value, 801 not supported,
 *     719 launch failed (CUresult numbering); the reason for the last
 *     non-zero return on the calling thread is pegainfer_kernels_last_error().
 *
 * Entry points named kimi_* keep the reference's symbol names, argument order
 * and shape guards (48 local experts, top-8, group 32), so they are drop-in
 * replacements.  Entry points named pega_* have no reference counterpart:
 * they are the shape-general forms (any expert count / top-k) used for the
 * dense and DeepSeek-V2-Lite-shaped configurations, plus the routing select
 * stages the reference runs inside larger calls or on the host.
 */
#ifndef PEGA_MOE_H_
#define PEGA_MOE_H_

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* Reason for the last failure on this thread (never NULL).
 * Replaces: pegainfer_kernels_last_error, pegainfer-kernels/csrc/shared/ffi_last_error.cu:13 */
const char* pegainfer_kernels_last_error(void);

/* ---------------- token -> expert permutation ---------------- */

/* Replaces kimi_moe_marlin_align_block_size_cuda, pegainfer-kernels/src/ffi/kimi.rs:279-294
 * (csrc/kimi_k2/kimi_experts.cu:197-268).  Deterministic for every route count. */
int kimi_moe_marlin_align_block_size_cuda(const int32_t* topk_idx, int32_t* sorted_token_ids,
                                          int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                          uint32_t* expert_offsets, uint32_t* expert_cursor,
                                          int active_tokens, int topk, int global_start,
                                          int local_experts, int block_size,
                                          int max_padded_tokens, int max_m_blocks,
                                          hipStream_t stream);

/* No reference counterpart: shape-general form of the call above (local_experts <= 512,
 * any topk). */
int pega_moe_align_block_size(const int32_t* topk_idx, int32_t* sorted_token_ids,
                              int32_t* expert_ids, int32_t* num_tokens_post_padded,
                              uint32_t* expert_offsets, uint32_t* expert_cursor,
                              int active_tokens, int topk, int global_start, int local_experts,
                              int block_size, int max_padded_tokens, int max_m_blocks,
                              hipStream_t stream);

/* Replaces kimi_deepep_build_marlin_routing_on_stream, pegainfer-kernels/src/ffi/kimi.rs:296-307
 * (csrc/kimi_k2/kimi_experts.cu:435-459). */
int kimi_deepep_build_marlin_routing_on_stream(const int32_t* psum_expert,
                                               int32_t* sorted_token_ids, int32_t* expert_ids,
                                               int32_t* num_tokens_post_padded,
                                               int num_local_experts, int alignment,
                                               int block_size, int max_padded_tokens,
                                               int max_m_blocks, hipStream_t stream);

/* ---------------- load-time weight packaging (Marlin layout, bit-exact) ---------------- */

/* Replaces kimi_marlin_int4_reorder_weight_cuda, pegainfer-kernels/src/ffi/kimi.rs:93-101. */
int kimi_marlin_int4_reorder_weight_cuda(const uint8_t* weight_packed_checkpoint,
                                         uint8_t* weight_packed_marlin, int in_dim, int out_dim,
                                         int local_experts, int group_size, hipStream_t stream);

/* Replaces kimi_marlin_int4_reorder_scale_cuda, pegainfer-kernels/src/ffi/kimi.rs:84-91. */
int kimi_marlin_int4_reorder_scale_cuda(const uint16_t* weight_scale_checkpoint,
                                        uint16_t* weight_scale_marlin, int in_dim, int out_dim,
                                        int local_experts, int group_size, hipStream_t stream);

/* Replaces kimi_marlin_int4_fuse_w13_cuda, pegainfer-kernels/src/ffi/kimi.rs:68-82. */
int kimi_marlin_int4_fuse_w13_cuda(const uint8_t* gate_weight_packed_marlin,
                                   const uint8_t* up_weight_packed_marlin,
                                   uint8_t* w13_weight_packed_marlin,
                                   const uint16_t* gate_scale_marlin,
                                   const uint16_t* up_scale_marlin, uint16_t* w13_scale_marlin,
                                   int in_dim, int intermediate_dim, int local_experts,
                                   int group_size, hipStream_t stream);

/* No reference counterpart: the three calls above for any expert count. */
int pega_marlin_int4_reorder_weight(const uint8_t* ckpt, uint8_t* marlin, int in_dim,
                                    int out_dim, int local_experts, int group_size,
                                    hipStream_t stream);
int pega_marlin_int4_reorder_scale(const uint16_t* ckpt, uint16_t* marlin, int in_dim,
                                   int out_dim, int local_experts, int group_size,
                                   hipStream_t stream);
int pega_marlin_int4_fuse_w13(const uint8_t* gate_w, const uint8_t* up_w, uint8_t* w13_w,
                              const uint16_t* gate_s, const uint16_t* up_s, uint16_t* w13_s,
                              int in_dim, int intermediate_dim, int local_experts,
                              int group_size, hipStream_t stream);

/* ---------------- grouped W4A16 GEMM ---------------- */

/* Replaces kimi_marlin_wna16_gemm_cuda, pegainfer-kernels/src/ffi/kimi.rs:131-152
 * (csrc/kimi_k2/kimi_marlin_wna16.cu:241-343,414-442).  c_tmp and workspace (locks) are
 * required as in the reference but not accessed: K is split inside each workgroup. */
int kimi_marlin_wna16_gemm_cuda(const uint16_t* input, uint16_t* output, float* c_tmp,
                                const uint8_t* b_qweight, const uint16_t* b_scales,
                                int32_t* workspace, const int32_t* sorted_token_ids,
                                const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                                const float* topk_weights, int workspace_len,
                                int sorted_token_ids_len, int moe_block_size, int top_k,
                                bool mul_topk_weights, int size_m, int size_n, int size_k,
                                int local_experts, int group_size, int sm_count,
                                hipStream_t stream);

/* No reference counterpart: shape-general form (any expert count; c_tmp / workspace unused
 * and may be NULL). */
int pega_wna16_gemm(const uint16_t* input, uint16_t* output, float* c_tmp, long long c_tmp_len,
                    const uint8_t* b_qweight, const uint16_t* b_scales, int32_t* workspace,
                    int workspace_len, const int32_t* sorted_token_ids, const int32_t* expert_ids,
                    const int32_t* num_tokens_post_padded, const float* topk_weights,
                    int sorted_token_ids_len, int moe_block_size, int top_k,
                    bool mul_topk_weights, int size_m, int size_n, int size_k, int local_experts,
                    int group_size, int sm_count, hipStream_t stream);

/* No reference counterpart: W13 GEMM fused with SwiGLU.  The reference runs
 * kimi_marlin_wna16_gemm_cuda (W13, top_k rows) then kimi_marlin_w13_swiglu_cuda over every
 * route row; here act = [size_m * top_k, intermediate_dim] bf16 gets SwiGLU of the W13 sums
 * rounded to bf16 as the W13 output is, for the routed rows only (other rows are left as they
 * are), and the W13 output never reaches HBM.  The bits are the pair's whenever both add the
 * fp32 products over the same K shares: always at block sizes 32-64 (one wave covers all of
 * K), and at block sizes 8/16 when the W13 GEMM has at least two workgroups per CU and K is at
 * least 512 (C3's decode layer, for one).  Otherwise the shares differ (the K split below, or
 * 8 waves where the GEMM runs 16), and the sums may differ from the pair's in the last fp32
 * bit, within the same summation error bound.
 *  - Block size 8 or 16 (decode): when the (block, tile) units are too few to fill the GPU
 *    (one expert at batch 1-8), K is split across workgroups; the fp32 partials (partials:
 *    at least 2 * size_m * top_k * 2 * intermediate_dim floats for a split, more allows more
 *    shares) are summed in share order by the SwiGLU kernel, which rounds gate and up to bf16
 *    exactly as the W13 output is rounded.  Otherwise (or when partials is NULL or too small
 *    to split) a workgroup takes a gate tile and its up tile and applies SwiGLU in its
 *    epilogue.
 *  - Block size 32, 48 or 64 (prefill): the tile GEMM (128-row tiles, or 64-row tiles when
 *    the routes fill at most 64 rows per expert on average) takes each gate tile and its up
 *    tile in one workgroup and applies SwiGLU in its epilogue; partials is not used (may be
 *    NULL, partials_len 0). */
int pega_wna16_w13_swiglu(const uint16_t* input, uint16_t* act, float* partials,
                          long long partials_len, const uint8_t* b_qweight,
                          const uint16_t* b_scales, const int32_t* sorted_token_ids,
                          const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                          int sorted_token_ids_len, int moe_block_size, int top_k, int size_m,
                          int intermediate_dim, int size_k, int local_experts, int group_size,
                          int sm_count, hipStream_t stream);

/* No reference counterpart; for callers that cannot allocate (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc): pega_wna16_w13_swiglu without the
 * partials workspace.  The K-split partials go to the library's static per-device scratch
 * (2 MiB = 524,288 floats, held until the process ends; its device address is looked up once
 * per device on the first call there).  Nothing in it needs clearing: every routed row of
 * every K share is written before the SwiGLU kernel reads it.  Calls that overlap on one
 * device race on the scratch.  The output is pega_wna16_w13_swiglu's with a partials
 * workspace of the scratch's size (partials_len = 524,288): the share count is capped by
 * what the scratch holds, and a wanted K split it cannot hold two shares of runs unsplit, as
 * the workspace entry does with a small workspace.  The current device must own `stream`
 * (status 1 otherwise). */
int pega_wna16_w13_swiglu_noalloc(const uint16_t* input, uint16_t* act, const uint8_t* b_qweight,
                                  const uint16_t* b_scales, const int32_t* sorted_token_ids,
                                  const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                                  int sorted_token_ids_len, int moe_block_size, int top_k,
                                  int size_m, int intermediate_dim, int size_k, int local_experts,
                                  int group_size, int sm_count, hipStream_t stream);

/* One problem of pega_wna16_prefill_pair: a grouped INT4 GEMM at a prefill block size (the
 * tile kernel), as pega_wna16_gemm (act NULL) or pega_wna16_w13_swiglu (act set) would run
 * it.  Plain pointers and sizes; 112 bytes on LP64. */
typedef struct pega_wna16_problem {
    const uint16_t* input;                /* bf16 [size_m, size_k], 16-byte aligned */
    uint16_t* output;                     /* bf16 [size_m * top_k, size_n] (unused with act) */
    uint16_t* act;                        /* non-NULL: SwiGLU epilogue into bf16
                                             [size_m * top_k, size_n / 2] */
    const uint8_t* b_qweight;             /* device-layout INT4 weights [local_experts] */
    const uint16_t* b_scales;             /* device-layout bf16 scales */
    const int32_t* sorted_token_ids;      /* the permutation of this problem's routes */
    const int32_t* expert_ids;
    const int32_t* num_tokens_post_padded;
    const float* topk_weights;            /* read only with mul_topk_weights */
    int sorted_token_ids_len;
    int moe_block_size;                   /* 32, 48 or 64 */
    int top_k;
    int mul_topk_weights;                 /* 0 or 1 (0 with act) */
    int size_m;
    int size_n;                           /* with act: 2 * intermediate_dim, gate then up */
    int size_k;
    int local_experts;
    int group_size;                       /* 32 */
} pega_wna16_problem;

/* No reference counterpart: two independent prefill-size GEMMs in one launch, e.g. a layer's
 * shared expert (first) and its routed experts (second).  The workgroups of the first problem
 * are dispatched first, and the second problem's fill the rest of the GPU, so one stream keeps
 * both running at once; each problem's output has the bits its own single launch gives.
 * Returns 801 when a problem's block size is 8 or 16 (the decode kernels). */
int pega_wna16_prefill_pair(const pega_wna16_problem* first, const pega_wna16_problem* second,
                            hipStream_t stream);

/* ---------------- activation / combine / residual ---------------- */

/* Replaces kimi_marlin_w13_swiglu_cuda, pegainfer-kernels/src/ffi/kimi.rs:113-119. */
int kimi_marlin_w13_swiglu_cuda(const uint16_t* w13, uint16_t* out, int rows,
                                int intermediate_dim, hipStream_t stream);

/* Replaces kimi_marlin_w13_swiglu_expanded_cuda, pegainfer-kernels/src/ffi/kimi.rs:121-129. */
int kimi_marlin_w13_swiglu_expanded_cuda(const uint16_t* w13, uint16_t* out,
                                         const int32_t* num_tokens_post_padded, int max_rows,
                                         int intermediate_dim, int sm_count, hipStream_t stream);

/* Replaces kimi_marlin_sum_topk_rows_f32_cuda, pegainfer-kernels/src/ffi/kimi.rs:104-111. */
int kimi_marlin_sum_topk_rows_f32_cuda(const uint16_t* route_output, float* out,
                                       int active_tokens, int topk, int hidden_dim,
                                       hipStream_t stream);

/* No reference C symbol: the DeepSeek-V2-Lite weighted fp32 combine (fmaf chain in route
 * order), restating pegainfer-kernels/csrc/deepseek_v2_lite/dsv2_lite_moe.cu:131-155. */
int pega_weighted_topk_sum_f32(const uint16_t* route_output, const float* topk_weight,
                               float* out, int active_tokens, int topk, int hidden_dim,
                               hipStream_t stream);

/* No reference counterpart: the top-k combine over the routes this GPU owns only
 * (topk_idx - global_start in [0, local_experts)); the other rows of route_output are not
 * read, so the caller skips their zero-fill (moe_nccl.rs:186-188).  topk_weight NULL: plain
 * sum as kimi_marlin_sum_topk_rows_f32_cuda; non-NULL: fmaf chain as
 * pega_weighted_topk_sum_f32.  Equal bit for bit to zero-filling the skipped rows and calling
 * those (for finite weights).  hidden_dim % 8 == 0, 16-byte aligned buffers. */
int pega_moe_combine_local_f32(const uint16_t* route_output, const int32_t* topk_idx,
                               const float* topk_weight, float* out, int active_tokens, int topk,
                               int hidden_dim, int global_start, int local_experts,
                               hipStream_t stream);

/* Replaces kimi_residual_add_scaled_f32_cuda, pegainfer-kernels/src/ffi/kimi.rs:309-317. */
int kimi_residual_add_scaled_f32_cuda(const uint16_t* hidden, const uint16_t* projected,
                                      const float* routed_f32, float scale, uint16_t* out, int n,
                                      hipStream_t stream);

/* Replaces kimi_residual_add_scaled_bf16_cuda, pegainfer-kernels/src/ffi/kimi.rs:319-327. */
int kimi_residual_add_scaled_bf16_cuda(const uint16_t* hidden, const uint16_t* projected,
                                       const uint16_t* routed, float scale, uint16_t* out, int n,
                                       hipStream_t stream);

/* Replaces kimi_add_f32_bf16_to_bf16_cuda, pegainfer-kernels/src/ffi/kimi.rs:9-15. */
int kimi_add_f32_bf16_to_bf16_cuda(const float* a, const uint16_t* b, uint16_t* out, int n,
                                   hipStream_t stream);

/* Replaces f32_to_bf16_cuda, pegainfer-kernels/src/ffi/shared.rs:849-854
 * (csrc/shared/elementwise.cu:235-244,722-728): out = bf16(input), round to nearest even. */
int f32_to_bf16_cuda(const float* input, uint16_t* output, int n, hipStream_t stream);

/* Replaces add_cuda, pegainfer-kernels/src/ffi/shared.rs:27-33
 * (csrc/shared/elementwise.cu:9-21,500-507): out = bf16(f(a) + f(b)). */
int add_cuda(const uint16_t* a, const uint16_t* b, uint16_t* out, int n, hipStream_t stream);

/* No reference symbol of its own: the DeepSeek-V2-Lite routed + shared join,
 * f32_to_bf16_cuda(routed) then add_cuda(., shared) as
 * pegainfer-deepseek-v2-lite/src/nccl_backend.rs:544-545 and runtime/moe.rs:656 run them,
 * in one pass with the same two roundings: out = bf16(f(bf16(routed)) + f(shared)). */
int pega_moe_join_routed_shared_bf16(const float* routed, const uint16_t* shared, uint16_t* out,
                                     int n, hipStream_t stream);

/* No reference symbol of its own: pega_moe_combine_local_f32 then
 * pega_moe_join_routed_shared_bf16 in one pass, for a layer whose routed sum needs no
 * reduction across GPUs between the two (one GPU holds every routed expert):
 * out[t] = bf16(f(bf16(combine_t)) + f(shared[t])), where combine_t is the fp32 sum (topk_weight
 * NULL) or fmaf chain over the token's local routes, k ascending from +0 -- the same bits as
 * the two calls.  hidden_dim % 8 == 0, 16-byte aligned buffers. */
int pega_moe_combine_join_bf16(const uint16_t* route_output, const int32_t* topk_idx,
                               const float* topk_weight, const uint16_t* shared, uint16_t* out,
                               int active_tokens, int topk, int hidden_dim, int global_start,
                               int local_experts, hipStream_t stream);

/* ---------------- dense bf16 GEMM (shared expert) ----------------
 * Y[n][m] = bf16(sum_k W[m][k] * X[n][k]) with fp32 accumulation; W [M][K],
 * X [N][K], Y [N][M] bf16 row-major (the reference's cublasGemmEx(OP_T, OP_N)
 * call, pegainfer-kernels/csrc/shared/linear.cu:321-344).  Needs M % 16 == 0,
 * K % 32 == 0 and 16-byte aligned W and X (801 otherwise).  Never allocates. */

/* Replaces gemm_cuda, pegainfer-kernels/src/ffi/shared.rs:220-228. */
int gemm_cuda(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
              hipStream_t stream);

/* Replaces gemm_graphsafe_cuda, pegainfer-kernels/src/ffi/shared.rs:230-238. */
int gemm_graphsafe_cuda(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                        hipStream_t stream);

/* No reference symbol of its own: gemm_graphsafe_cuda on the shared expert's gate/up weights
 * W13 [2 inter][K] (gate rows first) followed by kimi_marlin_w13_swiglu_cuda on its bf16 output,
 * as pegainfer-kimi-k2/src/runner/moe_nccl.rs:107-123 runs them, in one launch with the same
 * bits: act[n][j] = SwiGLU(bf16 gate sum, bf16 up sum).  X [N][K], act [N][inter].  Needs
 * inter % 16 == 0, K % 32 == 0 and 16-byte aligned W13 and X (801 otherwise).  Never
 * allocates. */
int pega_dense_w13_swiglu(const uint16_t* W13, const uint16_t* X, uint16_t* act, int inter, int N,
                          int K, hipStream_t stream);

/* ---------------- routing select ---------------- */

/* Replaces kimi_k2_router_noaux_tc_cuda, pegainfer-kernels/src/ffi/kimi.rs:52-66
 * (csrc/kimi_k2/kimi_router.cu:108-187): logits [padded_tokens][n_experts] fp32 =
 * hidden [padded_tokens][hidden_dim] . gate_weight [n_experts][hidden_dim]^T (fp32
 * accumulation), then the select stage below over the first active_tokens rows.  Same
 * rejections as the reference (1: null pointers, token counts, n_experts != 384,
 * topk != 8, route_scale <= 0); 801 when hidden_dim % 32 != 0 or hidden / gate_weight are
 * not 16-byte aligned. */
int kimi_k2_router_noaux_tc_cuda(const uint16_t* hidden, const uint16_t* gate_weight,
                                 const float* e_score_correction_bias, float* logits,
                                 float* topk_weight, int32_t* topk_idx, int active_tokens,
                                 int padded_tokens, int hidden_dim, int n_experts, int topk,
                                 float route_scale, hipStream_t stream);

/* No reference symbol of its own: the select stage (sigmoid, top-k of score+bias, renormalise)
 * of kimi_k2_router_noaux_tc_cuda, pegainfer-kernels/src/ffi/kimi.rs:52-66
 * (csrc/kimi_k2/kimi_router.cu:20-91), taking precomputed fp32 logits. */
int pega_kimi_router_select(const float* logits, const float* e_score_correction_bias,
                            float* topk_weight, int32_t* topk_idx, int active_tokens,
                            int n_experts, int topk, float route_scale, hipStream_t stream);

/* No reference symbol of its own: the router's select stage followed by the token -> expert
 * permutation, in one launch (the router fused into the permutation:
 * csrc/kimi_k2/kimi_router.cu:20-91 then csrc/kimi_k2/kimi_experts.cu:197-268, the pair
 * experts.rs:508-848 issues).  Outputs equal pega_kimi_router_select followed by
 * pega_moe_align_block_size (topk_idx / topk_weight over active_tokens rows, then the
 * permutation of their active_tokens * topk routes), bit for bit, with the union of those two
 * entry points' checks (status 1), and at most 4096 routes (801 above: a decode batch).  Above
 * four tokens the select runs in several workgroups and the last to finish sorts; they count
 * themselves in on a library-wide per-device counter, so launches of this entry point or of
 * pega_dsv2_route_align that overlap on one device race. */
int pega_kimi_route_align(const float* logits, const float* e_score_correction_bias,
                          float* topk_weight, int32_t* topk_idx, int32_t* sorted_token_ids,
                          int32_t* expert_ids, int32_t* num_tokens_post_padded,
                          uint32_t* expert_offsets, uint32_t* expert_cursor, int active_tokens,
                          int n_experts, int topk, float route_scale, int global_start,
                          int local_experts, int block_size, int max_padded_tokens,
                          int max_m_blocks, hipStream_t stream);

/* No reference counterpart: the routers' e^x, y[i] = the double-precision exp of x[i] rounded
 * to fp32, computed as the router kernels compute it (a double polynomial, falling back to the
 * double exp near fp32 rounding midpoints).  For tests that check it over every float. */
int pega_exp_exact_f32(const float* x, float* y, long long n, hipStream_t stream);

/* No reference symbol of its own: the DeepSeek-V2-Lite router (softmax top-k ordered by expert
 * id: pegainfer-deepseek-v2-lite/src/host_ops.rs:388-412, csrc/dsv2_lite/dsv2_lite_moe.cu:41-129)
 * followed by the token -> expert permutation, in one launch.  Outputs equal
 * pega_dsv2_router_select followed by pega_moe_align_block_size, bit for bit; the checks and
 * limits of pega_kimi_route_align (at most 4096 routes, 801 above), and the same race between
 * overlapping launches on one device. */
int pega_dsv2_route_align(const float* logits, float* topk_weight, int32_t* topk_idx,
                          int32_t* sorted_token_ids, int32_t* expert_ids,
                          int32_t* num_tokens_post_padded, uint32_t* expert_offsets,
                          uint32_t* expert_cursor, int tokens, int n_experts, int topk,
                          int global_start, int local_experts, int block_size,
                          int max_padded_tokens, int max_m_blocks, hipStream_t stream);

/* No reference C symbol: DeepSeek-V2-Lite softmax top-k sorted by expert id, restating
 * pegainfer-deepseek-v2-lite/src/host_ops.rs:388-412. */
int pega_dsv2_router_select(const float* logits, float* topk_weight, int32_t* topk_idx,
                            int tokens, int n_experts, int topk, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PEGA_MOE_H_ */
