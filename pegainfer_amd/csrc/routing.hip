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
// atomic cursor, so the order inside an expert varies run to run.  Both paths
// here are deterministic at every size.  Below 2048 routes it is one launch
// of one workgroup: each of the 16 waves owns a contiguous run of 64-route
// steps; inside a step the lanes holding the same expert find each other with
// one ballot per bit of the expert id, so a lane's rank among them is a
// popcount.  Per-(wave, expert) counts in LDS are scanned down the wave axis
// and across experts, and the scatter replays every step in order -- a
// stable counting sort, bit-exact with the contract.  From 2048 routes one
// launch of one workgroup per expert, and from 4096 a count launch and a
// scatter launch with one workgroup per expert, produce the same bytes (the
// per-expert and wide paths below).
#include "align_core.h"
#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

__global__ __launch_bounds__(kAlignThreads) void align_block_size_kernel(
    const int32_t* __restrict__ topk_idx, int32_t* __restrict__ sorted_token_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_tokens_post_padded,
    uint32_t* __restrict__ expert_offsets, uint32_t* __restrict__ expert_cursor,
    int route_elems, int global_start, int local_experts, int block_size,
    int max_padded_tokens, int max_m_blocks) {
  extern __shared__ __align__(16) unsigned char lds[];
  auto expert_of = [&](int r) {
    if (r >= route_elems) return -1;
    const int e = topk_idx[r] - global_start;
    return (e >= 0 && e < local_experts) ? e : -1;
  };
  align_workgroup(expert_of, lds, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  expert_offsets, expert_cursor, route_elems, local_experts, block_size,
                  max_padded_tokens, max_m_blocks);
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

// Wide path for large route counts: one workgroup per local expert, each
// scanning every route for its own expert id, so each route costs one compare
// and one ballot per expert instead of a ballot per id bit, and the work
// spreads over E compute units.  The route ids stay in L2 (4 B a route).
// Launch 1 counts each expert's routes into expert_cursor (its final value);
// launch 2 turns the counts into padded segment starts and writes each
// expert's segment in ascending route order: the same stable contract as the
// single-workgroup kernel, so both produce the same bytes.

// Routes in 64-route steps [s0, s1) whose id is `key` (wave-uniform result).
__device__ __forceinline__ int wave_count_key(const int32_t* __restrict__ topk_idx, int route_elems,
                                              int key, int s0, int s1) {
  const int lane = threadIdx.x & 63;
  int n = 0;
  for (int s = s0; s < s1; s += kAlignBatch) {
    int v[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      const int r = (s + j) * 64 + lane;
      v[j] = (s + j < s1 && r < route_elems) ? topk_idx[r] : -1;
    }
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) n += __popcll(__ballot(v[j] == key));
  }
  return n;
}

// This wave's share of the 64-route steps: waves own contiguous runs so that
// a wave's matches follow every match of the waves before it.
__device__ __forceinline__ void wave_steps(int route_elems, int& s0, int& s1) {
  const int steps = ceil_div(route_elems, 64);
  const int per_wave = ceil_div(steps, kAlignWaves);
  s0 = min((threadIdx.x >> 6) * per_wave, steps);
  s1 = min(s0 + per_wave, steps);
}

__global__ __launch_bounds__(kAlignThreads) void align_count_kernel(
    const int32_t* __restrict__ topk_idx, uint32_t* __restrict__ expert_cursor, int route_elems,
    int global_start) {
  __shared__ int s_n[kAlignWaves];
  int s0, s1;
  wave_steps(route_elems, s0, s1);
  const int n = wave_count_key(topk_idx, route_elems, global_start + static_cast<int>(blockIdx.x),
                               s0, s1);
  if ((threadIdx.x & 63) == 0) s_n[threadIdx.x >> 6] = n;
  __syncthreads();
  if (threadIdx.x == 0) {
    int total = 0;
    for (int w = 0; w < kAlignWaves; ++w) total += s_n[w];
    expert_cursor[blockIdx.x] = static_cast<uint32_t>(total);
  }
}

__global__ __launch_bounds__(kAlignThreads) void align_scatter_kernel(
    const int32_t* __restrict__ topk_idx, int32_t* __restrict__ sorted_token_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_tokens_post_padded,
    uint32_t* __restrict__ expert_offsets, const uint32_t* __restrict__ expert_cursor,
    int route_elems, int global_start, int local_experts, int block_size, int max_padded_tokens,
    int max_m_blocks) {
  __shared__ int s_before[kAlignWaves], s_total[kAlignWaves], s_n[kAlignWaves];
  const int e = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int key = global_start + e;
  // the counts' loads go out with the recount's
  const int count_t = t < local_experts ? static_cast<int>(expert_cursor[t]) : 0;
  const int count = static_cast<int>(expert_cursor[e]);
  int s0, s1;
  wave_steps(route_elems, s0, s1);
  const int n = wave_count_key(topk_idx, route_elems, key, s0, s1);

  // padded segment sizes of all experts (thread t holds expert t): this
  // segment's start is the sum over experts below e, the total over all
  const int padded = ceil_div(count_t, block_size) * block_size;
  int below_e = t < e ? padded : 0, all = padded;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    below_e += __shfl_xor(below_e, d, 64);
    all += __shfl_xor(all, d, 64);
  }
  if (lane == 0) {
    s_before[wave] = below_e;
    s_total[wave] = all;
    s_n[wave] = n;
  }
  __syncthreads();
  int start = 0, total = 0, rank = 0;
  for (int w = 0; w < kAlignWaves; ++w) {
    start += s_before[w];
    total += s_total[w];
    rank += w < wave ? s_n[w] : 0;
  }
  const int seg_end = start + ceil_div(count, block_size) * block_size;

  // this wave's matches in ascending route order, after the earlier waves'
  const uint64_t below = (1ull << lane) - 1ull;
  for (int s = s0; s < s1; s += kAlignBatch) {
    int v[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      const int r = (s + j) * 64 + lane;
      v[j] = (s + j < s1 && r < route_elems) ? topk_idx[r] : -1;
    }
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      const bool hit = v[j] == key;
      const uint64_t m = __ballot(hit);
      const int pos = start + rank + __popcll(m & below);
      if (hit && pos < max_padded_tokens) sorted_token_ids[pos] = (s + j) * 64 + lane;
      rank += __popcll(m);
    }
  }

  // the segment's padding and block ids; the tail past the total is shared
  // out over the whole grid
  for (int q = start + count + t; q < seg_end && q < max_padded_tokens; q += kAlignThreads)
    sorted_token_ids[q] = route_elems;
  for (int b = start / block_size + t; b < seg_end / block_size && b < max_m_blocks;
       b += kAlignThreads)
    expert_ids[b] = e;
  const int g = e * kAlignThreads + t, gstride = gridDim.x * kAlignThreads;
  for (int q = total + g; q < max_padded_tokens; q += gstride) sorted_token_ids[q] = route_elems;
  for (int b = total / block_size + g; b < max_m_blocks; b += gstride) expert_ids[b] = -1;
  if (t == 0) {
    expert_offsets[e] = static_cast<uint32_t>(start);
    if (e == 0) {
      expert_offsets[local_experts] = static_cast<uint32_t>(total);
      num_tokens_post_padded[0] = total;
    }
  }
}

// One launch, one workgroup per local expert: each workgroup first counts
// every expert's routes itself (per 64-route step, the lanes holding the same
// expert find each other by one ballot per id bit and the lowest of them adds
// the set's size to an LDS histogram), so no second launch has to wait for
// the counts; then it writes its own expert's segment as the scatter kernel
// above does.  Same bytes as the other two paths.
__global__ __launch_bounds__(kAlignThreads) void align_expert_kernel(
    const int32_t* __restrict__ topk_idx, int32_t* __restrict__ sorted_token_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_tokens_post_padded,
    uint32_t* __restrict__ expert_offsets, uint32_t* __restrict__ expert_cursor,
    int route_elems, int global_start, int local_experts, int block_size, int max_padded_tokens,
    int max_m_blocks) {
  __shared__ uint32_t s_hist[kAlignMaxExperts];
  __shared__ int s_before[kAlignWaves], s_total[kAlignWaves], s_n[kAlignWaves];
  const int e = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int E = local_experts;
  const int key = global_start + e;
  for (int i = t; i < E; i += kAlignThreads) s_hist[i] = 0;
  int s0, s1;
  wave_steps(route_elems, s0, s1);
  const int nbits = 32 - __builtin_clz(static_cast<unsigned>(max(E - 1, 1)));
  const uint64_t below = (1ull << lane) - 1ull;
  // the wave's ids stay in registers when its steps fit one batch
  const bool one_batch = s1 - s0 <= kAlignBatch;  // wave-uniform
  int v_keep[kAlignBatch];
  __syncthreads();

  int n = 0;  // this wave's routes of expert e
  for (int s = s0; s < s1; s += kAlignBatch) {
    int v[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      const int r = (s + j) * 64 + lane;
      v[j] = (s + j < s1 && r < route_elems) ? topk_idx[r] : -1;
      v_keep[j] = v[j];
    }
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      if (s + j >= s1) continue;  // wave-uniform
      const int le = v[j] - global_start;
      const int ex = (v[j] >= 0 && le >= 0 && le < E) ? le : -1;
      const uint64_t peers = same_expert_lanes(ex, nbits);
      if (ex >= 0 && (peers & below) == 0)
        atomicAdd(&s_hist[ex], static_cast<uint32_t>(__popcll(peers)));
      n += __popcll(__ballot(v[j] == key));
    }
  }
  __syncthreads();

  // padded segment sizes of all experts: this segment's start is the sum over
  // the experts below e, the total over all
  int below_e = 0, all = 0, count = 0;
  for (int i = t; i < E; i += kAlignThreads) {
    const int c = static_cast<int>(s_hist[i]);
    const int padded = ceil_div(c, block_size) * block_size;
    below_e += i < e ? padded : 0;
    all += padded;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    below_e += __shfl_xor(below_e, d, 64);
    all += __shfl_xor(all, d, 64);
  }
  if (lane == 0) {
    s_before[wave] = below_e;
    s_total[wave] = all;
    s_n[wave] = n;
  }
  __syncthreads();
  int start = 0, total = 0, rank = 0;
  for (int w = 0; w < kAlignWaves; ++w) {
    start += s_before[w];
    total += s_total[w];
    rank += w < wave ? s_n[w] : 0;
    count += s_n[w];
  }
  const int seg_end = start + ceil_div(count, block_size) * block_size;

  // this wave's routes of expert e in ascending route order, after the
  // earlier waves'
  for (int s = s0; s < s1; s += kAlignBatch) {
    int v[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      const int r = (s + j) * 64 + lane;
      v[j] = one_batch ? v_keep[j] : ((s + j < s1 && r < route_elems) ? topk_idx[r] : -1);
    }
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      if (s + j >= s1) continue;  // wave-uniform
      const bool hit = v[j] == key;
      const uint64_t m = __ballot(hit);
      const int pos = start + rank + __popcll(m & below);
      if (hit && pos < max_padded_tokens) sorted_token_ids[pos] = (s + j) * 64 + lane;
      rank += __popcll(m);
    }
  }

  // the segment's padding and block ids; the tail past the total is shared
  // out over the whole grid
  for (int q = start + count + t; q < seg_end && q < max_padded_tokens; q += kAlignThreads)
    sorted_token_ids[q] = route_elems;
  for (int b = start / block_size + t; b < seg_end / block_size && b < max_m_blocks;
       b += kAlignThreads)
    expert_ids[b] = e;
  const int g = e * kAlignThreads + t, gstride = gridDim.x * kAlignThreads;
  for (int q = total + g; q < max_padded_tokens; q += gstride) sorted_token_ids[q] = route_elems;
  for (int b = total / block_size + g; b < max_m_blocks; b += gstride) expert_ids[b] = -1;
  if (t == 0) {
    expert_offsets[e] = static_cast<uint32_t>(start);
    expert_cursor[e] = static_cast<uint32_t>(count);
    if (e == 0) {
      expert_offsets[E] = static_cast<uint32_t>(total);
      num_tokens_post_padded[0] = total;
    }
  }
}

// Route counts from which the per-expert path replaces the single workgroup
// (below it the one launch is shorter than two).
#ifndef PEGA_ALIGN_WIDE_MIN_ROUTES
#define PEGA_ALIGN_WIDE_MIN_ROUTES 4096
#endif
// From this many routes up to the wide path, the one-launch per-expert kernel
// (graph-timed, 64 experts, 3072 routes: 7.3 against 8.5 us for the single
// workgroup; it loses below ~2000 routes and against the two wide launches at
// 32768 routes, 25 against 14 us, where every workgroup's full histogram costs
// more than the second launch).
#ifndef PEGA_ALIGN_EXPERT_MIN_ROUTES
#define PEGA_ALIGN_EXPERT_MIN_ROUTES 2048
#endif

// Shape-general permutation (local_experts <= 512, any topk); the Kimi
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
  if (route_elems >= PEGA_ALIGN_EXPERT_MIN_ROUTES && route_elems < PEGA_ALIGN_WIDE_MIN_ROUTES) {
    hipLaunchKernelGGL(align_expert_kernel, dim3(local_experts), dim3(kAlignThreads), 0, stream,
                       topk_idx, sorted_token_ids, expert_ids, num_tokens_post_padded,
                       expert_offsets, expert_cursor, route_elems, global_start, local_experts,
                       block_size, max_padded_tokens, max_m_blocks);
    return launch_status("align_block_size");
  }
  if (route_elems >= PEGA_ALIGN_WIDE_MIN_ROUTES) {
    hipLaunchKernelGGL(align_count_kernel, dim3(local_experts), dim3(kAlignThreads), 0, stream,
                       topk_idx, expert_cursor, route_elems, global_start);
    hipLaunchKernelGGL(align_scatter_kernel, dim3(local_experts), dim3(kAlignThreads), 0, stream,
                       topk_idx, sorted_token_ids, expert_ids, num_tokens_post_padded,
                       expert_offsets, expert_cursor, route_elems, global_start, local_experts,
                       block_size, max_padded_tokens, max_m_blocks);
    return launch_status("align_block_size");
  }
  const size_t lds = align_lds_bytes(local_experts);
  hipLaunchKernelGGL(align_block_size_kernel, dim3(1), dim3(kAlignThreads), lds, stream, topk_idx,
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
// 48 experts and top-8); local_experts <= 512.  Used for the DeepSeek-V2-Lite
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

// Reference: pegainfer-kernels/src/ffi/kimi.rs:296-307; kimi_experts.cu:435-459,
// including its rejection of more than 64 local experts (:446, status 1).
PEGA_API int kimi_deepep_build_marlin_routing_on_stream(
    const int32_t* psum_expert, int32_t* sorted_token_ids, int32_t* expert_ids,
    int32_t* num_tokens_post_padded, int num_local_experts, int alignment, int block_size,
    int max_padded_tokens, int max_m_blocks, hipStream_t stream) {
  if (num_local_experts > 64)
    return pega::fail(pega::kInvalidValue,
                      "kimi deepep_build_routing: at most 64 local experts (got %d)",
                      num_local_experts);
  return pega::deepep_build_routing(psum_expert, sorted_token_ids, expert_ids,
                                    num_tokens_post_padded, num_local_experts, alignment,
                                    block_size, max_padded_tokens, max_m_blocks, stream);
}
