// The single-workgroup stable counting sort behind the token -> expert
// permutation, shared by the permutation kernel (routing.hip) and the fused
// router + permutation kernel (router.hip).  Device code only.
//
// One workgroup of 16 waves.  Each wave owns a contiguous run of 64-route
// steps; inside a step the lanes holding the same expert find each other with
// one ballot per bit of the expert id, so a lane's rank among them is a
// popcount.  Per-(wave, expert) counts in LDS are scanned down the wave axis
// and across experts, and the scatter replays every step in order: the
// order of experts.rs:1689-1717 (ascending expert, ascending route inside an
// expert, each segment padded to a multiple of block_size with the sentinel
// route_elems; expert_ids[b] = e per block, -1 past the total).
#pragma once

#include "common.h"

namespace pega {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxExperts = 512;  // one thread per expert; counts take 16 x 512 x 4 B of LDS
constexpr int kAlignBatch = 16;        // 64-route steps whose loads are in flight together

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

// Lanes of the wave holding the same local expert as this lane (valid lanes
// only; the result is meaningless on a lane with e < 0).  One ballot per bit
// of the id: a lane stays in the set while every bit agrees.
__device__ __forceinline__ uint64_t same_expert_lanes(int e, int nbits) {
  uint64_t m = __ballot(e >= 0);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t ones = __ballot(bit);
    m &= bit ? ones : ~ones;
  }
  return m;
}

// LDS the workgroup sort needs for E local experts: per-(wave, expert)
// counts, the segment starts and the per-wave totals.
inline size_t align_lds_bytes(int local_experts) {
  return sizeof(uint32_t) * kAlignWaves * local_experts +
         sizeof(int) * (local_experts + 1 + kAlignWaves);
}

// The sort over routes 0 .. route_elems - 1.  expert_of(r) returns route r's
// local expert or -1 (not local, or r past the end); every thread of the
// workgroup calls this, and `lds` holds align_lds_bytes(local_experts) bytes.
template <typename ExpertOf>
__device__ __forceinline__ void align_workgroup(
    ExpertOf expert_of, unsigned char* lds, int32_t* __restrict__ sorted_token_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ num_tokens_post_padded,
    uint32_t* __restrict__ expert_offsets, uint32_t* __restrict__ expert_cursor,
    int route_elems, int local_experts, int block_size, int max_padded_tokens,
    int max_m_blocks) {
  const int E = local_experts;
  uint32_t* cnt = reinterpret_cast<uint32_t*>(lds);       // [waves][E]
  int* seg_start = reinterpret_cast<int*>(cnt + kAlignWaves * E);  // [E + 1]
  int* wave_total = seg_start + (E + 1);                    // [waves]
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;

  for (int i = t; i < kAlignWaves * E; i += kAlignThreads) cnt[i] = 0;
  const int steps = ceil_div(route_elems, 64);
  const int per_wave = ceil_div(steps, kAlignWaves);
  const int s0 = min(wave * per_wave, steps), s1 = min(s0 + per_wave, steps);
  const int nbits = 32 - __builtin_clz(static_cast<unsigned>(max(E - 1, 1)));
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t* my_cnt = cnt + wave * E;
  __syncthreads();

  // 1. per-(wave, expert) route counts; the lowest lane of each peer set adds
  //    the set's size (peer sets have distinct experts, so no two lanes write
  //    one counter).  When the wave's steps fit one batch (up to 16 steps a
  //    wave, 16384 routes) their experts and peer sets stay in registers for
  //    the scatter, which then re-reads nothing.
  const bool one_batch = s1 - s0 <= kAlignBatch;  // wave-uniform
  int e_keep[kAlignBatch];
  uint64_t peers_keep[kAlignBatch];
  for (int s = s0; s < s1; s += kAlignBatch) {
    int e[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) e[j] = s + j < s1 ? expert_of((s + j) * 64 + lane) : -1;
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      e_keep[j] = e[j];
      peers_keep[j] = 0;
      if (s + j < s1) {  // wave-uniform
        const uint64_t peers = same_expert_lanes(e[j], nbits);
        peers_keep[j] = peers;
        if (e[j] >= 0 && (peers & below) == 0)
          my_cnt[e[j]] += static_cast<uint32_t>(__popcll(peers));
      }
    }
  }
  __syncthreads();

  // 2. thread e: exclusive scan of its column down the waves (the column
  //    becomes each wave's starting rank), then the padded exclusive scan of
  //    the segment sizes across experts
  int count = 0;
  if (t < E) {
    // all sixteen counts in flight first, then the scan in registers
    uint32_t c[kAlignWaves];
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) c[w] = cnt[w * E + t];
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) {
      cnt[w * E + t] = run;
      run += c[w];
    }
    count = static_cast<int>(run);
  }
  const int padded = ceil_div(count, block_size) * block_size;
  const int incl = wave_incl_scan(padded);
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  int before = 0, total = 0;
  for (int w = 0; w < kAlignWaves; ++w) {
    const int v = wave_total[w];
    before += w < wave ? v : 0;
    total += v;
  }
  if (t < E) {
    const int start = before + incl - padded;
    seg_start[t] = start;
    expert_offsets[t] = static_cast<uint32_t>(start);
    expert_cursor[t] = static_cast<uint32_t>(count);
    // sentinels on this segment's padding, and the expert of each of its blocks
    for (int q = start + count; q < start + padded && q < max_padded_tokens; ++q)
      sorted_token_ids[q] = route_elems;
    for (int b = start / block_size; b < (start + padded) / block_size && b < max_m_blocks; ++b)
      expert_ids[b] = t;
  }
  if (t == 0) {
    seg_start[E] = total;
    expert_offsets[E] = static_cast<uint32_t>(total);
    num_tokens_post_padded[0] = total;
  }
  __syncthreads();

  // 3. stable scatter: replay the steps in order; a lane's slot is its
  //    segment start + the wave's running rank + its rank among its peers,
  //    and the lowest peer then advances the running rank
  for (int s = s0; s < s1; s += kAlignBatch) {
    int e[kAlignBatch];
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j)
      e[j] = one_batch ? e_keep[j] : (s + j < s1 ? expert_of((s + j) * 64 + lane) : -1);
#pragma unroll
    for (int j = 0; j < kAlignBatch; ++j) {
      if (s + j >= s1) continue;  // wave-uniform
      const uint64_t peers = one_batch ? peers_keep[j] : same_expert_lanes(e[j], nbits);
      if (e[j] >= 0) {
        const uint32_t base = my_cnt[e[j]];
        const int pos = seg_start[e[j]] + static_cast<int>(base) + __popcll(peers & below);
        if (pos < max_padded_tokens) sorted_token_ids[pos] = (s + j) * 64 + lane;
        if ((peers & below) == 0) my_cnt[e[j]] = base + static_cast<uint32_t>(__popcll(peers));
      }
    }
  }

  // 4. sentinels past the total; no expert past it (each segment's blocks were
  //    written by their expert's thread above)
  for (int q = total + t; q < max_padded_tokens; q += kAlignThreads) sorted_token_ids[q] = route_elems;
  for (int blk = total / block_size + t; blk < max_m_blocks; blk += kAlignThreads)
    expert_ids[blk] = -1;
}


}  // namespace pega
