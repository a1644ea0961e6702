// Routing front of the expert path: turns router logits into (topk_idx,
// topk_weight), the input of the token -> expert permutation.
//
//   pega_kimi_router_select   sigmoid scores, top-k of score + bias (ties ->
//       lower id) kept in selection order, weight = score * (scale / sum).
//       Reference: pegainfer-kernels/csrc/kimi_k2/kimi_router.cu:20-91
//       (router_scores_topk_normalize_kernel; the logits GEMM before it,
//       :108-142, is cuBLAS and is not part of this library).
//   pega_dsv2_router_select   softmax (max-subtracted, sequential sum,
//       divide), top-k by probability (ties -> lower id), then ordered by
//       expert id; weight = probability.
//       Reference: pegainfer-deepseek-v2-lite/src/host_ops.rs:388-447.
//
// Scores use e^x rounded from a double-precision exp, so that the CPU checker
// reproduces them bit for bit and the selected indices agree exactly.
#include "common.h"

namespace pega {
namespace {

constexpr int kMaxPerLane = 16;  // n_experts <= 64 * 16

struct Best {
  float v;
  int i;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ Best wave_argmax(Best b) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    float ov = __shfl_xor(b.v, d, 64);
    int oi = __shfl_xor(b.i, d, 64);
    if (better(ov, oi, b.v, b.i)) { b.v = ov; b.i = oi; }
  }
  return b;
}

// One wave per token; lane l owns experts l, l+64, ...
__global__ void kimi_router_select_kernel(const float* __restrict__ logits,
                                          const float* __restrict__ bias,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk, float route_scale) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  float score[kMaxPerLane], choice[kMaxPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + 64 * j;
    if (e < n_experts) {
      const float l = logits[static_cast<long long>(t) * n_experts + e];
      score[j] = 1.0f / (1.0f + exp_exact_f32(-l));
      choice[j] = score[j] + bias[e];
    } else {
      score[j] = 0.0f;
      choice[j] = -__builtin_inff();
    }
  }
  float sum = 0.0f;
  float my_w = 0.0f;  // lane r keeps selection r
  int my_i = 0;
  for (int r = 0; r < topk; ++r) {
    Best b{-__builtin_inff(), n_experts};
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      if (e < n_experts && better(choice[j], e, b.v, b.i)) { b.v = choice[j]; b.i = e; }
    }
    b = wave_argmax(b);
    float s = 0.0f;
    if (b.i < n_experts) {
      const int owner = b.i & 63, slot = b.i >> 6;
      float mine = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxPerLane; ++j)
        if (j == slot) mine = score[j];
      s = __shfl(mine, owner, 64);
      if (lane == owner) {
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j)
          if (j == slot) choice[j] = -__builtin_inff();
      }
    }
    if (lane == r) { my_w = s; my_i = b.i; }
    sum += s;
  }
  const float scale = sum > 0.0f ? route_scale / sum : 0.0f;
  if (lane < topk) {
    topk_idx[t * topk + lane] = my_i;
    topk_weight[t * topk + lane] = my_w * scale;
  }
}

__global__ void dsv2_router_select_kernel(const float* __restrict__ logits,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  float p[kMaxPerLane];
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < n_experts ? logits[static_cast<long long>(t) * n_experts + e] : -__builtin_inff();
    mx = fmaxf(mx, p[j]);
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j)
    p[j] = (lane + 64 * j < n_experts) ? exp_exact_f32(p[j] - mx) : 0.0f;
  // Sequential fp32 sum over experts 0, 1, 2, ... (the reference's order).
  float sum = 0.0f;
  for (int e = 0; e < n_experts; ++e) {
    float mine = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
      if (j == (e >> 6)) mine = p[j];
    sum += __shfl(mine, e & 63, 64);
  }
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) p[j] = sum == 0.0f ? 0.0f : p[j] / sum;
  int my_i = 0x7fffffff;  // lane r keeps selection r
  float my_w = 0.0f;
  for (int r = 0; r < topk; ++r) {
    Best b{-__builtin_inff(), n_experts};
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + 64 * j;
      if (e < n_experts && better(p[j], e, b.v, b.i)) { b.v = p[j]; b.i = e; }
    }
    b = wave_argmax(b);
    float w = 0.0f;
    if (b.i < n_experts) {
      const int owner = b.i & 63, slot = b.i >> 6;
      float mine = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxPerLane; ++j)
        if (j == slot) mine = p[j];
      w = __shfl(mine, owner, 64);
      if (lane == owner) {
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j)
          if (j == slot) p[j] = -__builtin_inff();
      }
    }
    if (lane == r) { my_i = b.i; my_w = w; }
  }
  // Order the selection by expert id: a lane's rank is the number of selected
  // ids below its own (selected ids are distinct).
  int rank = 0;
  for (int r = 0; r < topk; ++r) {
    const int other = __shfl(my_i, r, 64);
    rank += (other < my_i) ? 1 : 0;
  }
  if (lane < topk) {
    topk_idx[t * topk + rank] = my_i;
    topk_weight[t * topk + rank] = my_w;
  }
}

constexpr int kWavesPerBlock = 4;

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
  hipLaunchKernelGGL(kimi_router_select_kernel, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream,
                     logits, e_score_correction_bias, topk_weight, topk_idx, active_tokens,
                     n_experts, topk, route_scale);
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
  hipLaunchKernelGGL(dsv2_router_select_kernel, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream,
                     logits, topk_weight, topk_idx, tokens, n_experts, topk);
  return launch_status("dsv2_router_select");
}
