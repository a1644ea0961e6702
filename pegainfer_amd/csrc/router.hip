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
#include "align_core.h"
#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

constexpr int kMaxPerLane = 16;  // n_experts <= 64 * 16
constexpr int kRouteAlignMaxRoutes = 4096;  // ids kept in LDS by the fused kernel

// Order-preserving map of a float to u32 (for non-NaN values; -0 is folded
// into +0 first, so equal floats give equal keys).  Key 0 lies below every
// real value and marks an empty or already selected slot.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// A DPP lane move with no "old" operand (bound_ctrl), so that the compiler folds
// it into the consuming max/min as a DPP source.  Rows outside kRowMask are not
// written by that fused instruction and keep their value, which is the value a
// max/min of the lane with itself would give.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, kRowMask, 0xF, true));
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

// Top-k of the wave's NS x 64 keys (expert id lane + 64 j), largest first,
// equal keys to the lower id.  Returns, on lane r < topk, the r-th selected
// id; the selected keys are cleared.  A round is one DPP max-reduction of the
// lanes' best keys; the holders of the maximum are a ballot, and only when
// several lanes hold it (equal keys) does a second reduction pick the lowest
// id (a lane's own slots are scanned from j = 0, so its candidate is its
// lowest id with that key).
template <int NS>
__device__ __forceinline__ int wave_topk_ids(uint32_t (&key)[NS], int lane, int topk) {
  int my_sel = 0;
  for (int r = 0; r < topk; ++r) {
    // the lane's best key and its lowest slot holding it, found before the
    // reduction so that they overlap its DPP latencies
    uint32_t best = key[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < NS; ++j) {
      const bool up = key[j] > best;
      best = up ? key[j] : best;
      bj = up ? j : bj;
    }
    const uint32_t top = wave_reduce_u32(best, MaxU32{});
    const bool mine = best == top;
    const uint64_t holders = __ballot(mine);
    int win;
    if (__popcll(holders) == 1) {
      const int wl = __builtin_ctzll(holders);
      win = __builtin_amdgcn_readlane(bj * 64 + lane, wl);
    } else {
      const uint32_t cand = mine ? static_cast<uint32_t>(bj * 64 + lane) : 0xffffffffu;
      win = static_cast<int>(wave_reduce_u32(cand, MinU32{}));
    }
    const int wj = win >> 6;
    if (lane == (win & 63)) {
#pragma unroll
      for (int j = 0; j < NS; ++j)
        if (j == wj) key[j] = 0;
    }
    if (lane == r) my_sel = win;
  }
  return my_sel;
}

// Token t's selection by one wave; lane l owns experts l, l+64, ... (NS slots
// per lane, NS * 64 >= n_experts).  The Kimi score of logit l is
// 1 / (1 + e^-l), e^-l rounded from a double exp.  Writes the token's top-k
// weights and returns, on lane r < topk, the r-th selected id (the caller
// stores the ids); lane r takes its expert's score from the owner lane once,
// after the rounds.
template <int NS>
__device__ __forceinline__ int kimi_select_token(const float* __restrict__ logits,
                                                 const float* __restrict__ bias,
                                                 float* __restrict__ topk_weight, int t,
                                                 int n_experts, int topk, float route_scale) {
  const int lane = threadIdx.x & 63;
  const float* row = logits + static_cast<long long>(t) * n_experts;
  // every slot's loads, then every slot's exponential side by side (the rare
  // double-precision fallbacks after), then the scores: kimi_score's bits
  float lg[NS], bi[NS], ex[NS], sc[NS];
  bool ok[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + 64 * j;
    lg[j] = e < n_experts ? row[e] : 0.0f;
    bi[j] = e < n_experts ? bias[e] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) ex[j] = exp_exact_f32_try(-lg[j], &ok[j]);
#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (!ok[j]) ex[j] = exp_exact_f32(-lg[j]);
  uint32_t key[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    sc[j] = 1.0f / (1.0f + ex[j]);
    key[j] = lane + 64 * j < n_experts ? order_key(sc[j] + bi[j]) : 0u;
  }
  const int my_i = wave_topk_ids<NS>(key, lane, topk);
  // the selected expert's score, from its owner lane's slot
  float my_s = 0.0f;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const float v = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute((my_i & 63) << 2, __builtin_bit_cast(int, sc[j])));
    if (j == (my_i >> 6)) my_s = v;
  }
  if (lane >= topk) my_s = 0.0f;
  // sum in selection order, as the reference's rounds add them
  float sum = 0.0f;
  for (int r = 0; r < topk; ++r) sum += lane_value(my_s, r);
  const float scale = sum > 0.0f ? route_scale / sum : 0.0f;
  if (lane < topk) topk_weight[t * topk + lane] = my_s * scale;
  return my_i;
}

// One wave per token.
template <int NS>
__global__ void kimi_router_select_kernel(const float* __restrict__ logits,
                                          const float* __restrict__ bias,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk, float route_scale) {
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave
  const int sel = kimi_select_token<NS>(logits, bias, topk_weight, t, n_experts, topk,
                                        route_scale);
  const int lane = static_cast<int>(threadIdx.x & 63);
  if (lane < topk) topk_idx[t * topk + lane] = sel;
}

// DeepSeek-V2-Lite selection of token t by one wave: softmax (max-subtracted,
// e^x rounded from a double exp, sum over experts 0, 1, 2, ... in order,
// divide), top-k by probability (equal to the lower id), then ordered by
// expert id.  Writes the weights; returns on lane r < topk the id of rank r
// in id order (lanes >= topk return 0x7fffffff).
template <int NS>
__device__ __forceinline__ int dsv2_select_token(const float* __restrict__ logits,
                                                 float* __restrict__ topk_weight, int t,
                                                 int n_experts, int topk) {
  const int lane = threadIdx.x & 63;
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
    p[j] = (lane + 64 * j < n_experts) ? exp_exact_f32_fast(p[j] - mx) : 0.0f;
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
  const int sel = wave_topk_ids<NS>(key, lane, topk);
  const int my_i = lane < topk ? sel : 0x7fffffff;
  // the selected probability, from its owner lane's slot
  float my_w = 0.0f;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const float v = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute((my_i & 63) << 2, __builtin_bit_cast(int, p[j])));
    if (j == (my_i >> 6)) my_w = v;
  }
  // Order the selection by expert id: a lane's rank is the number of selected
  // ids below its own (selected ids are distinct).
  int rank = 0;
  for (int r = 0; r < topk; ++r)
    rank += __builtin_amdgcn_readlane(my_i, r) < my_i ? 1 : 0;
  if (lane < topk) topk_weight[t * topk + rank] = my_w;
  // hand rank r's id to lane r
  int by_rank = 0x7fffffff;
  for (int r = 0; r < topk; ++r) {
    const int rr = __builtin_amdgcn_readlane(rank, r);
    const int id = __builtin_amdgcn_readlane(my_i, r);
    if (lane == rr) by_rank = id;
  }
  return by_rank;
}

template <int NS>
__global__ void dsv2_router_select_kernel(const float* __restrict__ logits,
                                          float* __restrict__ topk_weight,
                                          int32_t* __restrict__ topk_idx, int tokens,
                                          int n_experts, int topk) {
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave
  const int id = dsv2_select_token<NS>(logits, topk_weight, t, n_experts, topk);
  const int lane = static_cast<int>(threadIdx.x & 63);
  if (lane < topk) topk_idx[t * topk + lane] = id;
}

// Arrivals of the fused router + permutation kernel's workgroups, per device.
// Zero between launches: the last workgroup of a launch resets it.  Launches
// that overlap on one device race on it.
__device__ uint32_t g_route_arrivals;

// The router's select stage and the token -> expert permutation in one launch.
// Workgroup b's wave w selects tokens b + G (w + 16 i) (G = gridDim.x) and
// stores their ids with device-scope atomic stores; the workgroup then counts
// itself in on g_route_arrivals.  The last workgroup to arrive loads every id
// with device-scope atomic loads, resets the counter and runs the
// permutation's counting sort (align_core.h).  No workgroup waits for another,
// and no device-wide fence is needed: the ids themselves are device-coherent
// (the L2 is per XCD; an agent-scope release would write the whole L2 back),
// and each workgroup's id stores are complete (s_waitcnt 0, then a barrier)
// before its arrival is counted.  With one workgroup the ids go through LDS
// only.  Outputs are those of the select kernel followed by the permutation
// kernel, bit for bit.
template <int NS, bool kDsv2>
__global__ __launch_bounds__(kAlignThreads) void route_align_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias,
    float* __restrict__ topk_weight, int32_t* topk_idx,
    int32_t* __restrict__ sorted_token_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ num_tokens_post_padded, uint32_t* __restrict__ expert_offsets,
    uint32_t* __restrict__ expert_cursor, int tokens, int n_experts, int topk,
    float route_scale, int global_start, int local_experts, int block_size,
    int max_padded_tokens, int max_m_blocks) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_last;
  const int route_elems = tokens * topk;
  int32_t* s_idx = reinterpret_cast<int32_t*>(lds);  // [route_elems]
  unsigned char* sort_lds = lds + ((route_elems * 4 + 15) & ~15);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = gridDim.x;
  for (int t = blockIdx.x + G * wave; t < tokens; t += G * kAlignWaves) {
    int sel;
    if constexpr (kDsv2) sel = dsv2_select_token<NS>(logits, topk_weight, t, n_experts, topk);
    else sel = kimi_select_token<NS>(logits, bias, topk_weight, t, n_experts, topk, route_scale);
    if (lane < topk) {
      if (G == 1) {
        s_idx[t * topk + lane] = sel;
        topk_idx[t * topk + lane] = sel;
      } else {
        __hip_atomic_store(&topk_idx[t * topk + lane], sel, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (G > 1) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's id stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&g_route_arrivals, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == static_cast<uint32_t>(G - 1);
      if (s_last)
        __hip_atomic_store(&g_route_arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    for (int r = threadIdx.x; r < route_elems; r += kAlignThreads)
      s_idx[r] = __hip_atomic_load(&topk_idx[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  auto expert_of = [&](int r) {
    if (r >= route_elems) return -1;
    const int e = s_idx[r] - global_start;
    return (e >= 0 && e < local_experts) ? e : -1;
  };
  align_workgroup(expert_of, sort_lds, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  expert_offsets, expert_cursor, route_elems, local_experts, block_size,
                  max_padded_tokens, max_m_blocks);
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

// Workgroups of the fused router + permutation: about four tokens each (one
// per SIMD), a single workgroup (ids through LDS only) up to four tokens.
inline int route_align_grid(int tokens) { return tokens <= 4 ? 1 : ceil_div(tokens, 4); }

template <bool kDsv2>
struct RouteAlignLaunchT {
  template <int NS>
  struct L {
    static void run(size_t lds, hipStream_t stream, const float* logits, const float* bias,
                    float* w, int32_t* idx, int32_t* sorted_token_ids, int32_t* expert_ids,
                    int32_t* ntp, uint32_t* expert_offsets, uint32_t* expert_cursor, int tokens,
                    int n_experts, int topk, float scale, int global_start, int local_experts,
                    int block_size, int max_padded_tokens, int max_m_blocks) {
      hipLaunchKernelGGL((route_align_kernel<NS, kDsv2>), dim3(route_align_grid(tokens)),
                         dim3(kAlignThreads), lds, stream, logits, bias, w, idx,
                         sorted_token_ids, expert_ids, ntp, expert_offsets, expert_cursor,
                         tokens, n_experts, topk, scale, global_start, local_experts,
                         block_size, max_padded_tokens, max_m_blocks);
    }
  };
};
template <int NS>
using KimiRouteAlignLaunch = RouteAlignLaunchT<false>::L<NS>;
template <int NS>
using Dsv2RouteAlignLaunch = RouteAlignLaunchT<true>::L<NS>;

template <int NS>
struct Dsv2Launch {
  static void run(dim3 grid, hipStream_t stream, const float* logits, float* w, int32_t* idx,
                  int tokens, int n_experts, int topk) {
    hipLaunchKernelGGL(dsv2_router_select_kernel<NS>, grid, dim3(64 * kWavesPerBlock), 0, stream,
                       logits, w, idx, tokens, n_experts, topk);
  }
};

// Checks shared by the two fused router + permutation entry points; returns the
// dynamic LDS size through *lds.
int route_align_checks(const char* name, const float* logits, const void* bias,
                       const float* topk_weight, const int32_t* topk_idx,
                       const int32_t* sorted_token_ids, const int32_t* expert_ids,
                       const int32_t* num_tokens_post_padded, const uint32_t* expert_offsets,
                       const uint32_t* expert_cursor, int active_tokens, int n_experts,
                       int topk, int global_start, int local_experts, int block_size,
                       int max_padded_tokens, int max_m_blocks, size_t* lds) {
  if (!logits || !bias || !topk_weight || !topk_idx || !sorted_token_ids || !expert_ids ||
      !num_tokens_post_padded || !expert_offsets || !expert_cursor)
    return fail(kInvalidValue, "%s: null pointer", name);
  if (active_tokens <= 0 || n_experts <= 0 || n_experts > 64 * kMaxPerLane || topk <= 0 ||
      topk > n_experts || topk > 64)
    return fail(kInvalidValue, "%s: bad shape tokens=%d experts=%d topk=%d", name,
                active_tokens, n_experts, topk);
  if (global_start < 0 || local_experts <= 0 || local_experts > kAlignMaxExperts)
    return fail(kInvalidValue, "%s: bad expert range start=%d E=%d", name, global_start,
                local_experts);
  if (!(block_size == 8 || (block_size >= 16 && block_size <= 64 && block_size % 16 == 0)))
    return fail(kInvalidValue, "%s: block_size %d not in {8,16,32,48,64}", name, block_size);
  const long long route_elems = static_cast<long long>(active_tokens) * topk;
  if (route_elems > kRouteAlignMaxRoutes)
    return fail(kNotSupported, "%s: %lld routes (at most %d in one workgroup)", name,
                route_elems, kRouteAlignMaxRoutes);
  const long long req_padded = route_elems + static_cast<long long>(local_experts) * (block_size - 1);
  const int required_blocks = ceil_div(static_cast<int>(req_padded), block_size);
  if (max_padded_tokens < req_padded || max_m_blocks < required_blocks)
    return fail(kInvalidValue, "%s: capacity too small (padded %d < %lld or blocks %d < %d)",
                name, max_padded_tokens, req_padded, max_m_blocks, required_blocks);
  *lds = ((static_cast<size_t>(route_elems) * 4 + 15) & ~static_cast<size_t>(15)) +
         align_lds_bytes(local_experts);
  return kSuccess;
}

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

// No reference counterpart: the routers' correctly rounded e^x
// (exp_exact_f32_fast) over n floats, so a test can hold it against the
// double-precision exp rounded to fp32 over every float it is used on.
namespace pega {
namespace {
__global__ void exp_exact_kernel(const float* __restrict__ x, float* __restrict__ y, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    y[i] = exp_exact_f32_fast(x[i]);
}
}  // namespace
}  // namespace pega

PEGA_API int pega_exp_exact_f32(const float* x, float* y, long long n, hipStream_t stream) {
  if (!x || !y || n < 0) return pega::fail(pega::kInvalidValue, "exp_exact_f32: bad arguments");
  if (n == 0) return pega::kSuccess;
  long long grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(pega::exp_exact_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     stream, x, y, n);
  return pega::launch_status("exp_exact_f32");
}

// The select stage and the token -> expert permutation in one launch (no
// reference counterpart as one symbol: kimi_router.cu:20-91 followed by
// kimi_experts.cu:197-268).  Same outputs, bit for bit, as
// pega_kimi_router_select followed by pega_moe_align_block_size, with the
// union of their argument checks; at most kRouteAlignMaxRoutes routes (decode
// batches), kNotSupported above.
PEGA_API int pega_kimi_route_align(const float* logits, const float* e_score_correction_bias,
                                   float* topk_weight, int32_t* topk_idx,
                                   int32_t* sorted_token_ids, int32_t* expert_ids,
                                   int32_t* num_tokens_post_padded, uint32_t* expert_offsets,
                                   uint32_t* expert_cursor, int active_tokens, int n_experts,
                                   int topk, float route_scale, int global_start,
                                   int local_experts, int block_size, int max_padded_tokens,
                                   int max_m_blocks, hipStream_t stream) {
  size_t lds = 0;
  int rc = pega::route_align_checks("kimi_route_align", logits, e_score_correction_bias,
                                    topk_weight, topk_idx, sorted_token_ids, expert_ids,
                                    num_tokens_post_padded, expert_offsets, expert_cursor,
                                    active_tokens, n_experts, topk, global_start, local_experts,
                                    block_size, max_padded_tokens, max_m_blocks, &lds);
  if (rc != kSuccess) return rc;
  if (!(route_scale > 0.0f))
    return fail(kInvalidValue, "kimi_route_align: route_scale must be positive");
  launch_slots<KimiRouteAlignLaunch>(n_experts, lds, stream, logits, e_score_correction_bias,
                                     topk_weight, topk_idx, sorted_token_ids, expert_ids,
                                     num_tokens_post_padded, expert_offsets, expert_cursor,
                                     active_tokens, n_experts, topk, route_scale, global_start,
                                     local_experts, block_size, max_padded_tokens, max_m_blocks);
  return launch_status("kimi_route_align");
}

// The DeepSeek-V2-Lite router (softmax top-k ordered by expert id) and the
// token -> expert permutation in one launch (no reference counterpart as one
// symbol: host_ops.rs:388-412 / dsv2_lite_moe.cu:41-129 followed by the
// permutation).  Same outputs, bit for bit, as pega_dsv2_router_select
// followed by pega_moe_align_block_size.
PEGA_API int pega_dsv2_route_align(const float* logits, float* topk_weight, int32_t* topk_idx,
                                   int32_t* sorted_token_ids, int32_t* expert_ids,
                                   int32_t* num_tokens_post_padded, uint32_t* expert_offsets,
                                   uint32_t* expert_cursor, int tokens, int n_experts, int topk,
                                   int global_start, int local_experts, int block_size,
                                   int max_padded_tokens, int max_m_blocks, hipStream_t stream) {
  size_t lds = 0;
  int rc = pega::route_align_checks("dsv2_route_align", logits, logits, topk_weight, topk_idx,
                                    sorted_token_ids, expert_ids, num_tokens_post_padded,
                                    expert_offsets, expert_cursor, tokens, n_experts, topk,
                                    global_start, local_experts, block_size, max_padded_tokens,
                                    max_m_blocks, &lds);
  if (rc != kSuccess) return rc;
  launch_slots<Dsv2RouteAlignLaunch>(n_experts, lds, stream, logits, nullptr, topk_weight,
                                     topk_idx, sorted_token_ids, expert_ids,
                                     num_tokens_post_padded, expert_offsets, expert_cursor,
                                     tokens, n_experts, topk, 1.0f, global_start, local_experts,
                                     block_size, max_padded_tokens, max_m_blocks);
  return launch_status("dsv2_route_align");
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
