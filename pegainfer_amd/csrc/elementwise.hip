// Bandwidth-bound stages of the expert path: SwiGLU, top-k row sums and the
// residual joins.  Each kernel restates the reference's rounding points
// exactly and moves 16 bytes per lane per access where shapes allow.
//
//   kimi_marlin_w13_swiglu_cuda           kimi_marlin_wna16.cu:345-361,444-460
//   kimi_marlin_w13_swiglu_expanded_cuda  kimi_marlin_wna16.cu:367-390,462-493
//   kimi_marlin_sum_topk_rows_f32_cuda    kimi_marlin_wna16.cu:392-408,495-513
//   kimi_residual_add_scaled_f32_cuda     kimi_experts.cu:25-39,287-306
//   kimi_residual_add_scaled_bf16_cuda    kimi_experts.cu:308-346
//   kimi_add_f32_bf16_to_bf16_cuda        kimi_experts.cu:15-23,270-285
//   pega_weighted_topk_sum_f32            dsv2_lite_moe.cu:131-155 (fmaf chain)
//   pega_moe_combine_local_f32            either combine over local routes only
//   f32_to_bf16_cuda                      shared/elementwise.cu:235-244,722-728
//   add_cuda                              shared/elementwise.cu:9-21,500-507
//   pega_moe_join_routed_shared_bf16      the two calls above in one pass
//   pega_moe_combine_join_bf16            pega_moe_combine_local_f32 then the join, one pass
#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

__device__ __forceinline__ void swiglu8(const uint16_t* __restrict__ row, uint16_t* __restrict__ out,
                                        int inter, int c8) {
  const uint4 g = *reinterpret_cast<const uint4*>(row + c8);
  const uint4 u = *reinterpret_cast<const uint4*>(row + inter + c8);
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t ow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t lo = swiglu_one(bf_lo(gw[i]), bf_lo(uw[i]));
    uint16_t hi = swiglu_one(bf_hi(gw[i]), bf_hi(uw[i]));
    ow[i] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
  }
  *reinterpret_cast<uint4*>(out + c8) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

// rows read from `rows_ptr` (device) when non-null, clamped to max_rows.
__global__ void swiglu_vec_kernel(const uint16_t* __restrict__ w13, uint16_t* __restrict__ out,
                                  int rows, const int32_t* __restrict__ rows_ptr, int inter) {
  int nrows = rows;
  if (rows_ptr) {
    nrows = rows_ptr[0];
    if (nrows <= 0) return;
    if (nrows > rows) nrows = rows;
  }
  const int per_row = inter >> 3;
  const long long total = static_cast<long long>(nrows) * per_row;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long r = idx / per_row;
    const int c8 = static_cast<int>(idx - r * per_row) * 8;
    swiglu8(w13 + r * 2 * inter, out + r * inter, inter, c8);
  }
}

__global__ void swiglu_scalar_kernel(const uint16_t* __restrict__ w13, uint16_t* __restrict__ out,
                                     int rows, const int32_t* __restrict__ rows_ptr, int inter) {
  int nrows = rows;
  if (rows_ptr) {
    nrows = rows_ptr[0];
    if (nrows <= 0) return;
    if (nrows > rows) nrows = rows;
  }
  const long long total = static_cast<long long>(nrows) * inter;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long r = idx / inter;
    const int c = static_cast<int>(idx - r * inter);
    const uint16_t* row = w13 + r * 2 * inter;
    out[idx] = swiglu_one(bf2f(row[c]), bf2f(row[inter + c]));
  }
}

// out[t, d] = ((0 + r0) + r1) + ... + r_{topk-1}  (fp32, k ascending).
__global__ void sum_topk_vec_kernel(const uint16_t* __restrict__ route, float* __restrict__ out,
                                    int tokens, int topk, int hidden) {
  const int per_row = hidden >> 3;
  const long long total = static_cast<long long>(tokens) * per_row;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long t = idx / per_row;
    const int d8 = static_cast<int>(idx - t * per_row) * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < topk; ++k) {
      const uint4 v = *reinterpret_cast<const uint4*>(route + (t * topk + k) * hidden + d8);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf_lo(w[i]);
        acc[2 * i + 1] += bf_hi(w[i]);
      }
    }
    float4* o = reinterpret_cast<float4*>(out + t * hidden + d8);
    o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

__global__ void sum_topk_scalar_kernel(const uint16_t* __restrict__ route, float* __restrict__ out,
                                       int tokens, int topk, int hidden) {
  const long long total = static_cast<long long>(tokens) * hidden;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long t = idx / hidden;
    const int d = static_cast<int>(idx - t * hidden);
    float acc = 0.0f;
    for (int k = 0; k < topk; ++k) acc += bf2f(route[(t * topk + k) * hidden + d]);
    out[idx] = acc;
  }
}

// out[t, d] = fma(f(r_k), w[t, k], ...) for k ascending, starting from 0.
__global__ void weighted_topk_sum_kernel(const uint16_t* __restrict__ route,
                                         const float* __restrict__ topk_weight,
                                         float* __restrict__ out, int tokens, int topk,
                                         int hidden) {
  const long long total = static_cast<long long>(tokens) * hidden;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long t = idx / hidden;
    const int d = static_cast<int>(idx - t * hidden);
    float acc = 0.0f;
    for (int k = 0; k < topk; ++k)
      acc = __builtin_fmaf(bf2f(route[(t * topk + k) * hidden + d]), topk_weight[t * topk + k], acc);
    out[idx] = acc;
  }
}

// Top-k combine over the routes this GPU owns: route (t, k) is read only when
// topk_idx[t*topk + k] - global_start lies in [0, local_experts).  Plain sum
// (weights == nullptr: acc += f(r_k)) or fmaf chain (acc = fma(f(r_k), w, acc)),
// k ascending from +0.  A skipped row would have added +0 (or fma(0, w, acc)
// with finite w), which never changes a sum that starts at +0, so the result
// equals the zero-filled full combine bit for bit.
//
// One workgroup per (token, 1024-column chunk): the token's expert ids and
// weights are uniform over the workgroup (scalar loads), every local row's
// 16-byte load is in flight before the first add, and each wave writes 2 KB
// of the fp32 row.  kTopk > 0 fixes top-k at compile time (6 and 8 here).
constexpr int kCombineThreads = 128;
constexpr int kCombineCols = kCombineThreads * 8;

// kJoin: instead of the fp32 row, write bf16(f(bf16(sum)) + f(shared)) to
// joined (the DeepSeek-V2-Lite routed + shared join, the same two roundings).
template <bool kWeighted, int kTopk, bool kJoin = false>
__global__ __launch_bounds__(kCombineThreads) void combine_local_rows_kernel(
    const uint16_t* __restrict__ route, const int32_t* __restrict__ topk_idx,
    const float* __restrict__ weights, float* __restrict__ out, int topk_rt, int hidden,
    int chunks, int global_start, int local_experts, const uint16_t* __restrict__ shared = nullptr,
    uint16_t* __restrict__ joined = nullptr) {
  constexpr int kMaxK = kTopk > 0 ? kTopk : 1;
  const int topk = kTopk > 0 ? kTopk : topk_rt;
  const long long t = blockIdx.x / chunks;
  const int d8 = (static_cast<int>(blockIdx.x - t * chunks) * kCombineThreads + threadIdx.x) * 8;
  if (d8 >= hidden) return;
  const int32_t* idx = topk_idx + t * topk;
  const uint16_t* rows = route + t * topk * hidden + d8;
  uint4 sv = make_uint4(0, 0, 0, 0);
  if (kJoin) sv = *reinterpret_cast<const uint4*>(shared + t * hidden + d8);  // in flight early
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](const uint4& v, float wk) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if (kWeighted) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = __builtin_fmaf(bf_lo(w[i]), wk, acc[2 * i]);
        acc[2 * i + 1] = __builtin_fmaf(bf_hi(w[i]), wk, acc[2 * i + 1]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf_lo(w[i]);
        acc[2 * i + 1] += bf_hi(w[i]);
      }
    }
  };
  if (kTopk > 0) {
    // ids (and weights) first, so that they arrive in one scalar load
    int id[kMaxK];
    float wt[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      id[k] = idx[k];
      wt[k] = kWeighted ? weights[t * topk + k] : 0.0f;
    }
    bool local[kMaxK];
    uint4 v[kMaxK];
#pragma unroll
    for (int k = 0; k < kMaxK; ++k) {
      local[k] = static_cast<unsigned>(id[k] - global_start) < static_cast<unsigned>(local_experts);
      v[k] = local[k] ? *reinterpret_cast<const uint4*>(rows + static_cast<long long>(k) * hidden)
                      : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kMaxK; ++k)
      if (local[k]) add(v[k], wt[k]);
  } else {
    for (int k = 0; k < topk; ++k) {
      if (static_cast<unsigned>(idx[k] - global_start) >= static_cast<unsigned>(local_experts))
        continue;
      add(*reinterpret_cast<const uint4*>(rows + static_cast<long long>(k) * hidden),
          kWeighted ? weights[t * topk + k] : 0.0f);
    }
  }
  if (kJoin) {
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t ow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = f2bf(__fadd_rn(bf2f(f2bf(acc[2 * j])), bf_lo(sw[j])));
      const uint16_t hi = f2bf(__fadd_rn(bf2f(f2bf(acc[2 * j + 1])), bf_hi(sw[j])));
      ow[j] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
    *reinterpret_cast<uint4*>(joined + t * hidden + d8) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    return;
  }
  float4* o = reinterpret_cast<float4*>(out + t * hidden + d8);
  o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

template <bool kWeighted, bool kJoin = false>
void launch_combine_local(const uint16_t* route, const int32_t* topk_idx, const float* weights,
                          float* out, int tokens, int topk, int hidden, int global_start,
                          int local_experts, hipStream_t stream, const uint16_t* shared = nullptr,
                          uint16_t* joined = nullptr) {
  const int chunks = ceil_div(hidden, kCombineCols);
  const dim3 grid(static_cast<unsigned>(static_cast<long long>(tokens) * chunks));
  if (topk == 8)
    hipLaunchKernelGGL((combine_local_rows_kernel<kWeighted, 8, kJoin>), grid,
                       dim3(kCombineThreads), 0, stream, route, topk_idx, weights, out, topk,
                       hidden, chunks, global_start, local_experts, shared, joined);
  else if (topk == 6)
    hipLaunchKernelGGL((combine_local_rows_kernel<kWeighted, 6, kJoin>), grid,
                       dim3(kCombineThreads), 0, stream, route, topk_idx, weights, out, topk,
                       hidden, chunks, global_start, local_experts, shared, joined);
  else
    hipLaunchKernelGGL((combine_local_rows_kernel<kWeighted, 0, kJoin>), grid,
                       dim3(kCombineThreads), 0, stream, route, topk_idx, weights, out, topk,
                       hidden, chunks, global_start, local_experts, shared, joined);
}

// out = bf16( routed*scale + f(bf16(f(hidden) + f(projected))) )
template <bool kRoutedBf16>
__global__ void residual_add_scaled_kernel(const uint16_t* __restrict__ hidden,
                                           const uint16_t* __restrict__ projected,
                                           const void* __restrict__ routed, float scale,
                                           uint16_t* __restrict__ out, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x) {
    const uint16_t rounded = f2bf(bf2f(hidden[i]) + bf2f(projected[i]));
    const float r = kRoutedBf16 ? bf2f(static_cast<const uint16_t*>(routed)[i])
                                : static_cast<const float*>(routed)[i];
    const float scaled = __fmul_rn(r, scale);
    out[i] = f2bf(__fadd_rn(scaled, bf2f(rounded)));
  }
}

__global__ void add_f32_bf16_kernel(const float* __restrict__ a, const uint16_t* __restrict__ b,
                                    uint16_t* __restrict__ out, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    out[i] = f2bf(__fadd_rn(a[i], bf2f(b[i])));
}

// out = bf16(x)  (pegainfer-kernels/csrc/shared/elementwise.cu:235-244)
__global__ void f32_to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ out,
                                   long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    out[i] = f2bf(x[i]);
}

// out = bf16(f(a) + f(b))  (pegainfer-kernels/csrc/shared/elementwise.cu:9-21)
__global__ void add_bf16_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                uint16_t* __restrict__ out, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    out[i] = f2bf(__fadd_rn(bf2f(a[i]), bf2f(b[i])));
}

// The DeepSeek-V2-Lite routed + shared join as the reference rounds it: the
// fp32 routed sum goes to bf16 first (f32_to_bf16_cuda, nccl_backend.rs:
// 544-545), then the bf16 add (add_cuda via add_batch, runtime/moe.rs:656):
//   out = bf16( f(bf16(routed)) + f(shared) ).
// Eight elements per thread, 16-byte shared/out and 2 x 16-byte routed I/O.
__global__ void join_routed_shared_vec_kernel(const float* __restrict__ routed,
                                              const uint16_t* __restrict__ shared,
                                              uint16_t* __restrict__ out, long long n8) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8;
       i += static_cast<long long>(gridDim.x) * blockDim.x) {
    const float4 r0 = reinterpret_cast<const float4*>(routed)[2 * i];
    const float4 r1 = reinterpret_cast<const float4*>(routed)[2 * i + 1];
    const uint4 sv = reinterpret_cast<const uint4*>(shared)[i];
    const float r[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t ow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = f2bf(__fadd_rn(bf2f(f2bf(r[2 * j])), bf_lo(sw[j])));
      const uint16_t hi = f2bf(__fadd_rn(bf2f(f2bf(r[2 * j + 1])), bf_hi(sw[j])));
      ow[j] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
    reinterpret_cast<uint4*>(out)[i] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

__global__ void join_routed_shared_kernel(const float* __restrict__ routed,
                                          const uint16_t* __restrict__ shared,
                                          uint16_t* __restrict__ out, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    out[i] = f2bf(__fadd_rn(bf2f(f2bf(routed[i])), bf2f(shared[i])));
}

constexpr int kThreads = 256;

unsigned grid_cap(long long work, int cap) {
  long long g = (work + kThreads - 1) / kThreads;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_swiglu(const uint16_t* w13, uint16_t* out, int rows, const int32_t* rows_ptr,
                  int inter, int grid_limit, hipStream_t stream) {
  const bool vec = inter % 8 == 0 && aligned16(w13) && aligned16(out);
  const long long work = static_cast<long long>(rows) * (vec ? inter / 8 : inter);
  const unsigned grid = grid_cap(work, grid_limit);
  if (vec)
    hipLaunchKernelGGL(swiglu_vec_kernel, dim3(grid), dim3(kThreads), 0, stream, w13, out, rows,
                       rows_ptr, inter);
  else
    hipLaunchKernelGGL(swiglu_scalar_kernel, dim3(grid), dim3(kThreads), 0, stream, w13, out,
                       rows, rows_ptr, inter);
  return launch_status("w13_swiglu");
}

}  // namespace
}  // namespace pega

using namespace pega;

// Reference: pegainfer-kernels/src/ffi/kimi.rs:113-119.
PEGA_API int kimi_marlin_w13_swiglu_cuda(const uint16_t* w13, uint16_t* out, int rows,
                                         int intermediate_dim, hipStream_t stream) {
  if (!w13 || !out || rows < 0 || intermediate_dim <= 0)
    return fail(kInvalidValue, "w13_swiglu: bad arguments");
  if (rows == 0) return kSuccess;
  return launch_swiglu(w13, out, rows, nullptr, intermediate_dim, 1 << 20, stream);
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:121-129 (rows read on device,
// clamped to max_rows; occupancy-sized grid of cu_count * 8 blocks).
PEGA_API int kimi_marlin_w13_swiglu_expanded_cuda(const uint16_t* w13, uint16_t* out,
                                                  const int32_t* num_tokens_post_padded,
                                                  int max_rows, int intermediate_dim,
                                                  int sm_count, hipStream_t stream) {
  if (!w13 || !out || !num_tokens_post_padded || max_rows < 0 || intermediate_dim <= 0)
    return fail(kInvalidValue, "w13_swiglu_expanded: bad arguments");
  if (max_rows == 0) return kSuccess;
  if (sm_count <= 0) sm_count = current_cu_count();
  if (sm_count <= 0) return fail(kInvalidValue, "w13_swiglu_expanded: no device");
  return launch_swiglu(w13, out, max_rows, num_tokens_post_padded, intermediate_dim,
                       sm_count * 8, stream);
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:104-111.
PEGA_API int kimi_marlin_sum_topk_rows_f32_cuda(const uint16_t* route_output, float* out,
                                                int active_tokens, int topk, int hidden_dim,
                                                hipStream_t stream) {
  if (!route_output || !out || active_tokens < 0 || topk <= 0 || hidden_dim <= 0)
    return fail(kInvalidValue, "sum_topk_rows: bad arguments");
  if (active_tokens == 0) return kSuccess;
  const bool vec = hidden_dim % 8 == 0 && aligned16(route_output) && aligned16(out);
  const long long work = static_cast<long long>(active_tokens) * (vec ? hidden_dim / 8 : hidden_dim);
  const unsigned grid = grid_cap(work, 1 << 20);
  if (vec)
    hipLaunchKernelGGL(sum_topk_vec_kernel, dim3(grid), dim3(kThreads), 0, stream, route_output,
                       out, active_tokens, topk, hidden_dim);
  else
    hipLaunchKernelGGL(sum_topk_scalar_kernel, dim3(grid), dim3(kThreads), 0, stream,
                       route_output, out, active_tokens, topk, hidden_dim);
  return launch_status("sum_topk_rows");
}

// Weighted fp32 combine of routed rows (DeepSeek-V2-Lite accumulate order);
// no reference counterpart with this signature (the reference accumulates
// one expert at a time, dsv2_lite_moe.cu:131-155, in the same per-token order).
PEGA_API int pega_weighted_topk_sum_f32(const uint16_t* route_output, const float* topk_weight,
                                        float* out, int active_tokens, int topk, int hidden_dim,
                                        hipStream_t stream) {
  if (!route_output || !topk_weight || !out || active_tokens < 0 || topk <= 0 || hidden_dim <= 0)
    return fail(kInvalidValue, "weighted_topk_sum: bad arguments");
  if (active_tokens == 0) return kSuccess;
  const unsigned grid = grid_cap(static_cast<long long>(active_tokens) * hidden_dim, 1 << 20);
  hipLaunchKernelGGL(weighted_topk_sum_kernel, dim3(grid), dim3(kThreads), 0, stream,
                     route_output, topk_weight, out, active_tokens, topk, hidden_dim);
  return launch_status("weighted_topk_sum");
}

// Top-k combine restricted to local routes (no reference counterpart: it
// replaces the zero-fill of the non-local rows, moe_nccl.rs:186-188, plus
// kimi_marlin_sum_topk_rows_f32_cuda or the weighted accumulate, with one
// kernel that does not read those rows).
PEGA_API int pega_moe_combine_local_f32(const uint16_t* route_output, const int32_t* topk_idx,
                                        const float* topk_weight, float* out, int active_tokens,
                                        int topk, int hidden_dim, int global_start,
                                        int local_experts, hipStream_t stream) {
  if (!route_output || !topk_idx || !out || active_tokens < 0 || topk <= 0 || hidden_dim <= 0 ||
      local_experts <= 0)
    return fail(kInvalidValue, "combine_local: bad arguments");
  if (hidden_dim % 8 != 0 || !aligned16(route_output) || !aligned16(out))
    return fail(kInvalidValue, "combine_local: hidden_dim %% 8 and 16-byte alignment required");
  if (active_tokens == 0) return kSuccess;
  if (static_cast<long long>(active_tokens) * ceil_div(hidden_dim, kCombineCols) > 0x7fffffffLL)
    return fail(kInvalidValue, "combine_local: tokens x column chunks overflows the grid");
  if (topk_weight)
    launch_combine_local<true>(route_output, topk_idx, topk_weight, out, active_tokens, topk,
                               hidden_dim, global_start, local_experts, stream);
  else
    launch_combine_local<false>(route_output, topk_idx, topk_weight, out, active_tokens, topk,
                                hidden_dim, global_start, local_experts, stream);
  return launch_status("combine_local");
}

// No reference symbol of its own: pega_moe_combine_local_f32 followed by
// pega_moe_join_routed_shared_bf16 (the DeepSeek-V2-Lite layer's weighted
// combine, then f32_to_bf16 and the bf16 add with the shared expert's output,
// nccl_backend.rs:544-545, runtime/moe.rs:656) in one pass, for a layer whose
// routed sum needs no reduction across GPUs in between: the same fp32 chain and
// the same two roundings, without the fp32 routed rows in HBM.
PEGA_API int pega_moe_combine_join_bf16(const uint16_t* route_output, const int32_t* topk_idx,
                                        const float* topk_weight, const uint16_t* shared,
                                        uint16_t* out, int active_tokens, int topk,
                                        int hidden_dim, int global_start, int local_experts,
                                        hipStream_t stream) {
  if (!route_output || !topk_idx || !shared || !out || active_tokens < 0 || topk <= 0 ||
      hidden_dim <= 0 || local_experts <= 0)
    return fail(kInvalidValue, "combine_join: bad arguments");
  if (hidden_dim % 8 != 0 || !aligned16(route_output) || !aligned16(shared) || !aligned16(out))
    return fail(kInvalidValue, "combine_join: hidden_dim %% 8 and 16-byte alignment required");
  if (active_tokens == 0) return kSuccess;
  if (static_cast<long long>(active_tokens) * ceil_div(hidden_dim, kCombineCols) > 0x7fffffffLL)
    return fail(kInvalidValue, "combine_join: tokens x column chunks overflows the grid");
  if (topk_weight)
    launch_combine_local<true, true>(route_output, topk_idx, topk_weight, nullptr, active_tokens,
                                     topk, hidden_dim, global_start, local_experts, stream,
                                     shared, out);
  else
    launch_combine_local<false, true>(route_output, topk_idx, topk_weight, nullptr, active_tokens,
                                      topk, hidden_dim, global_start, local_experts, stream,
                                      shared, out);
  return launch_status("combine_join");
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:309-317.
PEGA_API int kimi_residual_add_scaled_f32_cuda(const uint16_t* hidden, const uint16_t* projected,
                                               const float* routed_f32, float scale, uint16_t* out,
                                               int n, hipStream_t stream) {
  if (!hidden || !projected || !routed_f32 || !out || n < 0)
    return fail(kInvalidValue, "residual_add_scaled_f32: bad arguments");
  if (n == 0) return kSuccess;
  hipLaunchKernelGGL(residual_add_scaled_kernel<false>, dim3(grid_cap(n, 1 << 20)),
                     dim3(kThreads), 0, stream, hidden, projected,
                     static_cast<const void*>(routed_f32), scale, out, static_cast<long long>(n));
  return launch_status("residual_add_scaled_f32");
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:319-327.
PEGA_API int kimi_residual_add_scaled_bf16_cuda(const uint16_t* hidden, const uint16_t* projected,
                                                const uint16_t* routed, float scale,
                                                uint16_t* out, int n, hipStream_t stream) {
  if (!hidden || !projected || !routed || !out || n < 0)
    return fail(kInvalidValue, "residual_add_scaled_bf16: bad arguments");
  if (n == 0) return kSuccess;
  hipLaunchKernelGGL(residual_add_scaled_kernel<true>, dim3(grid_cap(n, 1 << 20)),
                     dim3(kThreads), 0, stream, hidden, projected,
                     static_cast<const void*>(routed), scale, out, static_cast<long long>(n));
  return launch_status("residual_add_scaled_bf16");
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:9-15.
PEGA_API int kimi_add_f32_bf16_to_bf16_cuda(const float* a, const uint16_t* b, uint16_t* out,
                                            int n, hipStream_t stream) {
  if (!a || !b || !out || n < 0) return fail(kInvalidValue, "add_f32_bf16: bad arguments");
  if (n == 0) return kSuccess;
  hipLaunchKernelGGL(add_f32_bf16_kernel, dim3(grid_cap(n, 1 << 20)), dim3(kThreads), 0, stream,
                     a, b, out, static_cast<long long>(n));
  return launch_status("add_f32_bf16");
}

// Reference: pegainfer-kernels/src/ffi/shared.rs:849-854 (f32_to_bf16_cuda,
// csrc/shared/elementwise.cu:722-728).
PEGA_API int f32_to_bf16_cuda(const float* input, uint16_t* output, int n, hipStream_t stream) {
  if (!input || !output || n < 0) return fail(kInvalidValue, "f32_to_bf16: bad arguments");
  if (n == 0) return kSuccess;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_cap(n, 1 << 20)), dim3(kThreads), 0, stream,
                     input, output, static_cast<long long>(n));
  return launch_status("f32_to_bf16");
}

// Reference: pegainfer-kernels/src/ffi/shared.rs:27-33 (add_cuda,
// csrc/shared/elementwise.cu:500-507).
PEGA_API int add_cuda(const uint16_t* a, const uint16_t* b, uint16_t* out, int n,
                      hipStream_t stream) {
  if (!a || !b || !out || n < 0) return fail(kInvalidValue, "add: bad arguments");
  if (n == 0) return kSuccess;
  hipLaunchKernelGGL(add_bf16_kernel, dim3(grid_cap(n, 1 << 20)), dim3(kThreads), 0, stream, a, b,
                     out, static_cast<long long>(n));
  return launch_status("add");
}

// No reference symbol of its own: f32_to_bf16_cuda(routed) followed by
// add_cuda(bf16 routed, shared), the DeepSeek-V2-Lite layer's routed + shared
// join (nccl_backend.rs:544-545, runtime/moe.rs:656), in one pass with the
// same two roundings.
PEGA_API int pega_moe_join_routed_shared_bf16(const float* routed, const uint16_t* shared,
                                              uint16_t* out, int n, hipStream_t stream) {
  if (!routed || !shared || !out || n < 0)
    return fail(kInvalidValue, "join_routed_shared: bad arguments");
  if (n == 0) return kSuccess;
  if (n % 8 == 0 && aligned16(routed) && aligned16(shared) && aligned16(out)) {
    const long long n8 = n / 8;
    hipLaunchKernelGGL(join_routed_shared_vec_kernel, dim3(grid_cap(n8, 1 << 20)),
                       dim3(kThreads), 0, stream, routed, shared, out, n8);
  } else {
    hipLaunchKernelGGL(join_routed_shared_kernel, dim3(grid_cap(n, 1 << 20)), dim3(kThreads), 0,
                       stream, routed, shared, out, static_cast<long long>(n));
  }
  return launch_status("join_routed_shared");
}
