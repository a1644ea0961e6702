// Routing front of the expert path: turns router logits into (topk_idx,
// topk_weight), the input of the token -> expert permutation.
//
//   pega_kimi_router_select   sigmoid scores, top-k of score + bias (ties ->
//       lower id) kept in selection order, weight = score * (scale / sum).
//       Reference: pegainfer-kernels/csrc/kimi_k2/kimi_router.cu:20-91
//       (router_scores_topk_normalize_kernel).
//   kimi_k2_router_noaux_tc_cuda   the logits GEMM (hidden x gate^T, fp32
//       out, kimi_router.cu:108-142, cuBLAS there, dense.hip's MFMA GEMM
//       here) followed by the select stage above, with the reference's
//       guards (kimi_router.cu:148-187).
//   pega_dsv2_router_select   softmax (max-subtracted, sequential sum,
//       divide), top-k by probability (ties -> lower id), then ordered by
//       expert id; weight = probability.
//       Reference: pegainfer-deepseek-v2-lite/src/host_ops.rs:388-447.
//
// Scores use e^x rounded from a double-precision exp, so that the CPU checker
// reproduces them bit for bit and the selected indices agree exactly.
#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

constexpr int kMaxPerLane = 16;  // n_experts <= 64 * 16

// Order-preserving map of a float to u32 (for non-NaN values; -0 is folded
// into +0 first, so equal floats give equal keys).  Key 0 lies below every
// real value and marks an empty or already selected slot.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      static_cast<int>(v), static_cast<int>(v), kCtrl, kRowMask, 0xF, false));
}

// Wave-wide reduction over DPP lane moves (quad swaps, half-row and row
// mirrors, then the row-15 and row-31 broadcasts); lane 63 ends up holding
// the result, which is read into a scalar register.
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, Op op) {
  v = op(v, dpp_mov<0xB1>(v));        // quad_perm [1,0,3,2]
  v = op(v, dpp_mov<0x4E>(v));        // quad_perm [2,3,0,1]
  v = op(v, dpp_mov<0x141>(v));       // row_half_mirror
  v = op(v, dpp_mov<0x140>(v));       // row_mirror
  v = op(v, dpp_mov<0x142, 0xA>(v));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_mov<0x143, 0xC>(v));  // row_bcast:31 into rows 2 and 3
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

struct MaxU32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
struct MinU32 {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; }
};

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Index of the largest key over the wave's NS x 64 slots, ties to the lower
// index (expert id lane + 64 j); the result is wave-uniform.
template <int NS>
__device__ __forceinline__ int wave_argmax(const uint32_t (&key)[NS], int lane) {
  uint32_t best = 0;
  int bj = 0;
#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (key[j] > best) { best = key[j]; bj = j; }  // strict: the lower slot keeps a tie
  const uint32_t top = wave_reduce_u32(best, MaxU32{});
  const uint32_t cand = best == top ? static_cast<uint32_t>(lane + 64 * bj) : 0xffffffffu;
  return static_cast<int>(wave_reduce_u32(cand, MinU32{}));
}

template <int NS>
__device__ __forceinline__ float slot_value(const float (&v)[NS], int slot) {
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (j == slot) r = v[j];
  return r;
}

// One wave per token; lane l owns experts l, l+64, ... (NS slots per lane,
// NS * 64 >= n_experts).
template <int NS>
__global__ void kimi_router_select_kernel(const float* __restrict__ logits,
                                          const float* __restrict__ bias,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk, float route_scale) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave
  float score[NS];
  uint32_t key[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + 64 * j;
    if (e < n_experts) {
      const float l = logits[static_cast<long long>(t) * n_experts + e];
      score[j] = 1.0f / (1.0f + exp_exact_f32(-l));
      key[j] = order_key(score[j] + bias[e]);
    } else {
      score[j] = 0.0f;
      key[j] = 0;
    }
  }
  float sum = 0.0f;
  float my_w = 0.0f;  // lane r keeps selection r
  int my_i = 0;
  for (int r = 0; r < topk; ++r) {
    const int sel = wave_argmax<NS>(key, lane);
    const int owner = sel & 63, slot = sel >> 6;
    const float s = lane_value(slot_value<NS>(score, slot), owner);
    if (lane == owner) {
#pragma unroll
      for (int j = 0; j < NS; ++j)
        if (j == slot) key[j] = 0;
    }
    if (lane == r) { my_w = s; my_i = sel; }
    sum += s;
  }
  const float scale = sum > 0.0f ? route_scale / sum : 0.0f;
  if (lane < topk) {
    topk_idx[t * topk + lane] = my_i;
    topk_weight[t * topk + lane] = my_w * scale;
  }
}

template <int NS>
__global__ void dsv2_router_select_kernel(const float* __restrict__ logits,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave
  float p[NS];
  uint32_t mkey = 0;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < n_experts ? logits[static_cast<long long>(t) * n_experts + e] : 0.0f;
    if (e < n_experts) mkey = max(mkey, order_key(p[j]));
  }
  mkey = wave_reduce_u32(mkey, MaxU32{});
  const float mx = __builtin_bit_cast(float, (mkey & 0x80000000u) ? (mkey & 0x7fffffffu) : ~mkey);
#pragma unroll
  for (int j = 0; j < NS; ++j)
    p[j] = (lane + 64 * j < n_experts) ? exp_exact_f32(p[j] - mx) : 0.0f;
  // Sequential fp32 sum over experts 0, 1, 2, ... (the reference's order).
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < NS; ++j)
    for (int l = 0; l < 64 && 64 * j + l < n_experts; ++l) sum += lane_value(p[j], l);
  uint32_t key[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    p[j] = sum == 0.0f ? 0.0f : p[j] / sum;
    key[j] = lane + 64 * j < n_experts ? order_key(p[j]) : 0;
  }
  int my_i = 0x7fffffff;  // lane r keeps selection r
  float my_w = 0.0f;
  for (int r = 0; r < topk; ++r) {
    const int sel = wave_argmax<NS>(key, lane);
    const int owner = sel & 63, slot = sel >> 6;
    const float w = lane_value(slot_value<NS>(p, slot), owner);
    if (lane == owner) {
#pragma unroll
      for (int j = 0; j < NS; ++j)
        if (j == slot) key[j] = 0;
    }
    if (lane == r) { my_i = sel; my_w = w; }
  }
  // Order the selection by expert id: a lane's rank is the number of selected
  // ids below its own (selected ids are distinct).
  int rank = 0;
  for (int r = 0; r < topk; ++r)
    rank += __builtin_amdgcn_readlane(my_i, r) < my_i ? 1 : 0;
  if (lane < topk) {
    topk_idx[t * topk + rank] = my_i;
    topk_weight[t * topk + rank] = my_w;
  }
}

constexpr int kWavesPerBlock = 4;

// Smallest compiled slot count covering n_experts (so the per-round scans do
// not walk empty slots: 6 for 384 experts, 1 for 64).
template <template <int> class Launch, typename... Args>
void launch_slots(int n_experts, Args... args) {
  const int need = ceil_div(n_experts, 64);
  if (need <= 1) Launch<1>::run(args...);
  else if (need <= 2) Launch<2>::run(args...);
  else if (need <= 4) Launch<4>::run(args...);
  else if (need <= 6) Launch<6>::run(args...);
  else if (need <= 8) Launch<8>::run(args...);
  else Launch<kMaxPerLane>::run(args...);
}

template <int NS>
struct KimiLaunch {
  static void run(dim3 grid, hipStream_t stream, const float* logits, const float* bias, float* w,
                  int32_t* idx, int tokens, int n_experts, int topk, float scale) {
    hipLaunchKernelGGL(kimi_router_select_kernel<NS>, grid, dim3(64 * kWavesPerBlock), 0, stream,
                       logits, bias, w, idx, tokens, n_experts, topk, scale);
  }
};

template <int NS>
struct Dsv2Launch {
  static void run(dim3 grid, hipStream_t stream, const float* logits, float* w, int32_t* idx,
                  int tokens, int n_experts, int topk) {
    hipLaunchKernelGGL(dsv2_router_select_kernel<NS>, grid, dim3(64 * kWavesPerBlock), 0, stream,
                       logits, w, idx, tokens, n_experts, topk);
  }
};

}  // namespace
}  // namespace pega

using namespace pega;

// The select stage of the Kimi noaux_tc router (no reference symbol of its
// own: it is the second half of kimi_k2_router_noaux_tc_cuda,
// pegainfer-kernels/src/ffi/kimi.rs:52-66).  Tokens past active_tokens are
// not written, as in the reference.
PEGA_API int pega_kimi_router_select(const float* logits, const float* e_score_correction_bias,
                                     float* topk_weight, int32_t* topk_idx, int active_tokens,
                                     int n_experts, int topk, float route_scale,
                                     hipStream_t stream) {
  if (!logits || !e_score_correction_bias || !topk_weight || !topk_idx)
    return fail(kInvalidValue, "kimi_router_select: null pointer");
  if (active_tokens <= 0 || n_experts <= 0 || n_experts > 64 * kMaxPerLane || topk <= 0 ||
      topk > n_experts || topk > 64 || !(route_scale > 0.0f))
    return fail(kInvalidValue, "kimi_router_select: bad shape tokens=%d experts=%d topk=%d",
                active_tokens, n_experts, topk);
  const unsigned grid = static_cast<unsigned>(ceil_div(active_tokens, kWavesPerBlock));
  launch_slots<KimiLaunch>(n_experts, dim3(grid), stream, logits, e_score_correction_bias,
                           topk_weight, topk_idx, active_tokens, n_experts, topk, route_scale);
  return launch_status("kimi_router_select");
}

// DeepSeek-V2-Lite softmax top-k (no reference C symbol: the reference runs
// this on the host, pegainfer-deepseek-v2-lite/src/host_ops.rs:388-412).
PEGA_API int pega_dsv2_router_select(const float* logits, float* topk_weight, int32_t* topk_idx,
                                     int tokens, int n_experts, int topk, hipStream_t stream) {
  if (!logits || !topk_weight || !topk_idx)
    return fail(kInvalidValue, "dsv2_router_select: null pointer");
  if (tokens <= 0 || n_experts <= 0 || n_experts > 64 * kMaxPerLane || topk <= 0 ||
      topk > n_experts || topk > 64)
    return fail(kInvalidValue, "dsv2_router_select: bad shape");
  const unsigned grid = static_cast<unsigned>(ceil_div(tokens, kWavesPerBlock));
  launch_slots<Dsv2Launch>(n_experts, dim3(grid), stream, logits, topk_weight, topk_idx, tokens,
                           n_experts, topk);
  return launch_status("dsv2_router_select");
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:52-66 (kimi_k2_router_noaux_tc_cuda,
// csrc/kimi_k2/kimi_router.cu:148-187): logits[padded_tokens][n_experts] =
// hidden[padded_tokens][hidden_dim] . gate_weight[n_experts][hidden_dim]^T in fp32
// (CUBLAS_COMPUTE_32F_PEDANTIC there: no reduced-precision accumulation; here fp32 MFMA
// accumulation, summed over K shares in a fixed order), then the select stage over the
// active tokens.  Same rejections as the reference (1 for null pointers, token counts,
// n_experts != 384, topk != 8, route_scale <= 0); additionally 801 when hidden_dim % 32 != 0
// or hidden / gate_weight are not 16-byte aligned (the MFMA GEMM's layout; Kimi-K2's
// hidden_dim is 7168).
PEGA_API int kimi_k2_router_noaux_tc_cuda(const uint16_t* hidden, const uint16_t* gate_weight,
                                          const float* e_score_correction_bias, float* logits,
                                          float* topk_weight, int32_t* topk_idx,
                                          int active_tokens, int padded_tokens, int hidden_dim,
                                          int n_experts, int topk, float route_scale,
                                          hipStream_t stream) {
  if (!hidden || !gate_weight || !e_score_correction_bias || !logits || !topk_weight || !topk_idx)
    return fail(kInvalidValue, "kimi_k2_router_noaux_tc: null pointer");
  if (active_tokens <= 0 || padded_tokens <= 0 || active_tokens > padded_tokens ||
      hidden_dim <= 0 || n_experts <= 0 || topk <= 0 || topk > n_experts || n_experts != 384 ||
      topk != 8 || !(route_scale > 0.0f))
    return fail(kInvalidValue,
                "kimi_k2_router_noaux_tc: bad shape active=%d padded=%d hidden=%d experts=%d "
                "topk=%d", active_tokens, padded_tokens, hidden_dim, n_experts, topk);
  const int rc = dense_gemm_f32(gate_weight, hidden, logits, n_experts, padded_tokens, hidden_dim,
                                stream, "kimi_k2_router_noaux_tc (logits)");
  if (rc != kSuccess) return rc;
  return pega_kimi_router_select(logits, e_score_correction_bias, topk_weight, topk_idx,
                                 active_tokens, n_experts, topk, route_scale, stream);
}
