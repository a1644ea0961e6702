// Token -> expert permutation and block metadata for the grouped expert GEMM.
//
//   kimi_moe_marlin_align_block_size_cuda  (reference: pegainfer-kernels/csrc/
//       kimi_k2/kimi_experts.cu:197-268, Rust op src/ops/kimi_k2/experts.rs:767-848)
//   kimi_deepep_build_marlin_routing_on_stream (kimi_experts.cu:369-459)
//
// The permutation contract (experts.rs:1689-1717): for each local expert in
// ascending order, its route offsets r (topk_idx[r] == global_start + e) are
// listed in ascending r, each segment padded to a multiple of block_size with
// the sentinel route_elems; expert_ids[b] = e for every block of the segment
// and -1 past the total.  The reference meets this order only on its
// single-block path (< 1024 routes); its 4-launch path takes positions from an
// atomic cursor, so the order inside an expert varies run to run.  This
// implementation is one deterministic launch for every size: each thread owns
// a contiguous run of routes, a per-(thread, expert) histogram in LDS is
// prefix-scanned down the thread axis, and the scatter walks every run in
// order again -- a stable counting sort, bit-exact with the contract.
#include "common.h"

namespace pega {
namespace {

constexpr int kAlignMaxThreads = 1024;
constexpr int kAlignMaxExperts = 224;  // 64 threads x 224 experts x 4 B fits the LDS budget
constexpr int kAlignLdsBudget = 56 * 1024;  // bytes of u32 per-thread histograms

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Largest e in [0, n) with start[e] <= p (start non-decreasing, start[0] = 0).
__device__ __forceinline__ int segment_of(const int* start, int n, int p) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (start[mid] <= p) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ void align_block_size_kernel(const int32_t* __restrict__ topk_idx,
                                        int32_t* __restrict__ sorted_token_ids,
                                        int32_t* __restrict__ expert_ids,
                                        int32_t* __restrict__ num_tokens_post_padded,
                                        uint32_t* __restrict__ expert_offsets,
                                        uint32_t* __restrict__ expert_cursor, int route_elems,
                                        int global_start, int local_experts, int block_size,
                                        int max_padded_tokens, int max_m_blocks) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int E = local_experts;
  const int T = blockDim.x;
  const int t = threadIdx.x;
  int* seg_start = reinterpret_cast<int*>(lds);         // [E + 1]
  int* count = seg_start + (E + 1);                      // [E]
  uint32_t* hist = reinterpret_cast<uint32_t*>(count + E);  // [T][E]

  const int chunk = (route_elems + T - 1) / T;
  const int r0 = min(t * chunk, route_elems);
  const int r1 = min(r0 + chunk, route_elems);
  uint32_t* my = hist + static_cast<size_t>(t) * E;
  for (int e = 0; e < E; ++e) my[e] = 0;
  for (int r = r0; r < r1; ++r) {
    int e = topk_idx[r] - global_start;
    if (e >= 0 && e < E) my[e] += 1;
  }
  __syncthreads();

  // Exclusive scan of hist[:, e] over threads; count[e] = column total.
  const int waves = T >> 6, wave = t >> 6, lane = t & 63;
  const int per_lane = T >> 6;  // T is a multiple of 64
  for (int e = wave; e < E; e += waves) {
    int run = 0;
    for (int i = 0; i < per_lane; ++i) run += static_cast<int>(hist[static_cast<size_t>(lane * per_lane + i) * E + e]);
    int incl = wave_incl_scan(run);
    int base = incl - run;
    for (int i = 0; i < per_lane; ++i) {
      uint32_t* cell = &hist[static_cast<size_t>(lane * per_lane + i) * E + e];
      int c = static_cast<int>(*cell);
      *cell = static_cast<uint32_t>(base);
      base += c;
    }
    if (lane == 63) count[e] = incl;
  }
  __syncthreads();

  // Padded exclusive scan over experts (wave 0).
  if (wave == 0) {
    const int per = (E + 63) / 64;
    int run = 0;
    for (int i = 0; i < per; ++i) {
      int e = lane * per + i;
      if (e < E) run += ceil_div(count[e], block_size) * block_size;
    }
    int incl = wave_incl_scan(run);
    int base = incl - run;
    for (int i = 0; i < per; ++i) {
      int e = lane * per + i;
      if (e < E) {
        seg_start[e] = base;
        expert_offsets[e] = static_cast<uint32_t>(base);
        expert_cursor[e] = static_cast<uint32_t>(count[e]);
        base += ceil_div(count[e], block_size) * block_size;
      }
    }
    if (lane == 63) {
      seg_start[E] = incl;
      expert_offsets[E] = static_cast<uint32_t>(incl);
      num_tokens_post_padded[0] = incl;
    }
  }
  __syncthreads();

  // Stable scatter: this thread's routes in order, after all earlier threads'.
  // The histogram row now holds the exclusive per-expert prefix.
  for (int r = r0; r < r1; ++r) {
    int e = topk_idx[r] - global_start;
    if (e >= 0 && e < E) {
      int pos = seg_start[e] + my[e];
      my[e] += 1;
      if (pos < max_padded_tokens) sorted_token_ids[pos] = r;
    }
  }
  // Sentinels on padding slots and past the total; expert id per block.
  const int total = seg_start[E];
  for (int p = t; p < max_padded_tokens; p += T) {
    if (p >= total) {
      sorted_token_ids[p] = route_elems;
    } else {
      int e = segment_of(seg_start, E, p);
      if (p - seg_start[e] >= count[e]) sorted_token_ids[p] = route_elems;
    }
  }
  for (int b = t; b < max_m_blocks; b += T) {
    int slot = b * block_size;
    expert_ids[b] = slot < total ? segment_of(seg_start, E, slot) : -1;
  }
}

// Metadata for an input that is already expert-major (the DeepEP receive
// buffer): psum_expert holds, per expert, the end of its rows, each expert's
// start being the previous end rounded up to `alignment`.
__global__ void deepep_routing_kernel(const int32_t* __restrict__ psum_expert,
                                      int32_t* __restrict__ sorted_token_ids,
                                      int32_t* __restrict__ expert_ids,
                                      int32_t* __restrict__ num_tokens_post_padded,
                                      int num_local_experts, int alignment, int block_size,
                                      int max_padded_tokens, int max_m_blocks) {
  extern __shared__ __align__(16) unsigned char lds[];
  int* start = reinterpret_cast<int*>(lds);
  int* count = start + num_local_experts;
  const int t = threadIdx.x;
  for (int e = t; e < num_local_experts; e += blockDim.x) {
    int s = 0;
    if (e > 0) s = ceil_div(psum_expert[e - 1], alignment) * alignment;
    int c = psum_expert[e] - s;
    start[e] = s;
    count[e] = c < 0 ? 0 : c;
  }
  __syncthreads();
  const int total = psum_expert[num_local_experts];
  for (int p = t; p < max_padded_tokens; p += blockDim.x) {
    int v = max_padded_tokens;
    if (p < total) {
      int e = segment_of(start, num_local_experts, p);
      if (p - start[e] < count[e]) v = p;
    }
    sorted_token_ids[p] = v;
  }
  for (int b = t; b < max_m_blocks; b += blockDim.x) {
    int slot = b * block_size;
    expert_ids[b] = slot < total ? segment_of(start, num_local_experts, slot) : 0;
  }
  if (t == 0) num_tokens_post_padded[0] = total;
}

bool valid_block_size(int bs) { return bs == 8 || (bs >= 16 && bs <= 64 && bs % 16 == 0); }

}  // namespace

// Shape-general permutation (local_experts <= 224, any topk); the Kimi
// entry point below adds the reference's fixed-shape guards.
int align_block_size(const int32_t* topk_idx, int32_t* sorted_token_ids, int32_t* expert_ids,
                     int32_t* num_tokens_post_padded, uint32_t* expert_offsets,
                     uint32_t* expert_cursor, int active_tokens, int topk, int global_start,
                     int local_experts, int block_size, int max_padded_tokens,
                     int max_m_blocks, hipStream_t stream) {
  if (!topk_idx || !sorted_token_ids || !expert_ids || !num_tokens_post_padded ||
      !expert_offsets || !expert_cursor)
    return fail(kInvalidValue, "align_block_size: null pointer");
  if (active_tokens <= 0 || topk <= 0 || global_start < 0 || local_experts <= 0 ||
      local_experts > kAlignMaxExperts)
    return fail(kInvalidValue, "align_block_size: bad shape tokens=%d topk=%d start=%d E=%d",
                active_tokens, topk, global_start, local_experts);
  if (!valid_block_size(block_size))
    return fail(kInvalidValue, "align_block_size: block_size %d not in {8,16,32,48,64}",
                block_size);
  const long long route_elems_ll = static_cast<long long>(active_tokens) * topk;
  const long long req_padded = route_elems_ll + static_cast<long long>(local_experts) * (block_size - 1);
  if (req_padded > 0x7fffffffLL)
    return fail(kInvalidValue, "align_block_size: route count overflows int32");
  const int route_elems = static_cast<int>(route_elems_ll);
  const int required_blocks = ceil_div(static_cast<int>(req_padded), block_size);
  if (max_padded_tokens < req_padded || max_m_blocks < required_blocks)
    return fail(kInvalidValue,
                "align_block_size: capacity too small (padded %d < %lld or blocks %d < %d)",
                max_padded_tokens, req_padded, max_m_blocks, required_blocks);
  int threads = kAlignMaxThreads;
  while (threads > 64 && static_cast<size_t>(threads) * local_experts * 4 > kAlignLdsBudget)
    threads >>= 1;
  const size_t lds = sizeof(int) * (2 * local_experts + 1) +
                     sizeof(uint32_t) * static_cast<size_t>(threads) * local_experts;
  hipLaunchKernelGGL(align_block_size_kernel, dim3(1), dim3(threads), lds, stream, topk_idx,
                     sorted_token_ids, expert_ids, num_tokens_post_padded, expert_offsets,
                     expert_cursor, route_elems, global_start, local_experts, block_size,
                     max_padded_tokens, max_m_blocks);
  return launch_status("align_block_size");
}

int deepep_build_routing(const int32_t* psum_expert, int32_t* sorted_token_ids,
                         int32_t* expert_ids, int32_t* num_tokens_post_padded,
                         int num_local_experts, int alignment, int block_size,
                         int max_padded_tokens, int max_m_blocks, hipStream_t stream) {
  if (!psum_expert || !sorted_token_ids || !expert_ids || !num_tokens_post_padded)
    return fail(kInvalidValue, "deepep_build_routing: null pointer");
  if (num_local_experts <= 0 || num_local_experts > 1024 || alignment <= 0 ||
      block_size <= 0 || max_padded_tokens < 0 || max_m_blocks < 0)
    return fail(kInvalidValue, "deepep_build_routing: bad shape");
  const size_t lds = sizeof(int) * 2 * num_local_experts;
  hipLaunchKernelGGL(deepep_routing_kernel, dim3(1), dim3(1024), lds, stream, psum_expert,
                     sorted_token_ids, expert_ids, num_tokens_post_padded, num_local_experts,
                     alignment, block_size, max_padded_tokens, max_m_blocks);
  return launch_status("deepep_build_routing");
}

}  // namespace pega

// ---------------------------------------------------------------- C ABI
// Reference: pegainfer-kernels/src/ffi/kimi.rs:279-294 (declaration),
// csrc/kimi_k2/kimi_experts.cu:197-230 (guards: topk == 8, local_experts == 48).
PEGA_API int kimi_moe_marlin_align_block_size_cuda(
    const int32_t* topk_idx, int32_t* sorted_token_ids, int32_t* expert_ids,
    int32_t* num_tokens_post_padded, uint32_t* expert_offsets, uint32_t* expert_cursor,
    int active_tokens, int topk, int global_start, int local_experts, int block_size,
    int max_padded_tokens, int max_m_blocks, hipStream_t stream) {
  if (topk != 8 || local_experts != 48)
    return pega::fail(pega::kInvalidValue,
                      "kimi align: requires topk == 8 and local_experts == 48 (got %d, %d)",
                      topk, local_experts);
  return pega::align_block_size(topk_idx, sorted_token_ids, expert_ids, num_tokens_post_padded,
                                expert_offsets, expert_cursor, active_tokens, topk,
                                global_start, local_experts, block_size, max_padded_tokens,
                                max_m_blocks, stream);
}

// Shape-general variant (no reference counterpart: the reference hard-codes
// 48 experts and top-8); local_experts <= 224.  Used for the DeepSeek-V2-Lite
// shape and one-expert cases.
PEGA_API int pega_moe_align_block_size(const int32_t* topk_idx, int32_t* sorted_token_ids,
                                       int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                       uint32_t* expert_offsets, uint32_t* expert_cursor,
                                       int active_tokens, int topk, int global_start,
                                       int local_experts, int block_size,
                                       int max_padded_tokens, int max_m_blocks,
                                       hipStream_t stream) {
  return pega::align_block_size(topk_idx, sorted_token_ids, expert_ids, num_tokens_post_padded,
                                expert_offsets, expert_cursor, active_tokens, topk,
                                global_start, local_experts, block_size, max_padded_tokens,
                                max_m_blocks, stream);
}

// Reference: pegainfer-kernels/src/ffi/kimi.rs:296-307; kimi_experts.cu:435-459
// (which limits num_local_experts to 64; this one allows up to 1024).
PEGA_API int kimi_deepep_build_marlin_routing_on_stream(
    const int32_t* psum_expert, int32_t* sorted_token_ids, int32_t* expert_ids,
    int32_t* num_tokens_post_padded, int num_local_experts, int alignment, int block_size,
    int max_padded_tokens, int max_m_blocks, hipStream_t stream) {
  return pega::deepep_build_routing(psum_expert, sorted_token_ids, expert_ids,
                                    num_tokens_post_padded, num_local_experts, alignment,
                                    block_size, max_padded_tokens, max_m_blocks, stream);
}
