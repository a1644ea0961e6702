// Grouped W4A16 expert GEMM on MI355X (gfx950): INT4 group-32 symmetric
// weights in the Marlin layout (see repack.hip), bf16 activations gathered by
// the token -> expert permutation, fp32 accumulation on MFMA 32x32x16 bf16.
//
// Semantics (reference: vendored Marlin, pegainfer-kernels/csrc/kimi_k2/
// vllm_marlin/moe/marlin_moe_wna16/marlin_template.h):
//   for every m-block b < ntp/bs of expert e = expert_ids[b], row i:
//     sid = sorted_token_ids[b*bs + i];  skip if sid >= size_m*top_k  (:466-537)
//     acc[n] = sum_k f(A[sid / top_k][k]) * f(bf16((q[e][n][k] - 8) * s[e][k/32][n]))
//              (dequant :112-124,1411-1413; MMA fp32 accumulate :1417-1426)
//     c = bf16(acc);  if mul_topk_weights: c = bf16(f(c) * f(bf16(topk_w[sid])))
//     C[sid][n] = c                                                (:1772-1900)
//
// Dequantisation is exact: the nibble v is placed in an fp16 whose value is
// 1024 + v (or 64 + v), v_fma_mix_f32 forms (1024 + v)*s - 1032*s = (v-8)*s
// with no rounding (every term fits fp32), and v_cvt_pk_bf16_f32 rounds that
// product to bf16 with round-to-nearest-even -- the same value as the
// reference's bf16 multiply q*s.
//
// Fragment map (per 64-column Marlin tile nt, per quant group g = k-tiles
// 2g, 2g+1): lane l -> column c = l%32, k-half h = l/32.  The lane owns
// columns n0 = nt*64 + (c/8)*16 + c%8 and n1 = n0 + 8, reads the four words
// (th = 4*(c%8) + jj, w = c/8), jj = 0..3, of tile (2g + h, nt), and feeds
// four MFMAs: X1/X2 (column n0, words jj in {0,1} / {2,3}) and Y1/Y2
// (column n1).  The activation lane (row m = l%32, h) supplies
// A[m][32g + 16h + {0..3, 8..11}] (X1/Y1) and {4..7, 12..15} (X2/Y2), i.e.
// one 32-byte read.  Scales of n0 and n1 are adjacent in the permuted scale
// row: index 8*(c%8) + 2*(c/8) (+1).
#include <algorithm>
#include <atomic>

#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16_t;

// (x & mask) | bits in plain C, never as a vector inline-asm statement: the
// compiler's hazard tracking cannot see VGPRs written inside asm, and a VALU
// write landing in the destination (or a source) of an MFMA still in flight
// is exactly the hazard it must see to insert wait states.  With `mask` in an
// SGPR this is one v_and_or_b32 (a VOP3 on gfx9 takes no literal operand, so
// with literal masks the compiler would emit v_and + v_or instead).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
  return (x & mask) | bits;
}

// The dequant constants in registers the compiler treats as opaque: the
// masks in SGPRs (s_mov_b32 in an asm statement that writes only SGPRs, which
// no MFMA reads) and the fp16 bias patterns in VGPRs (a DPP move of a
// wave-uniform value, which the compiler does not fold).  v_and_or_b32 then
// takes one SGPR and one VGPR operand, within gfx9's one-scalar-operand limit.
struct DqConst {
  uint32_t m_lo, m_hi;  // 0x000F000F, 0x00F000F0
  uint32_t k1024, k64;  // fp16 1024 | 1024 and 64 | 64
};
__device__ __forceinline__ DqConst dq_consts() {
  uint32_t lo, hi;
  asm("s_mov_b32 %0, 0x000f000f" : "=s"(lo));
  asm("s_mov_b32 %0, 0x00f000f0" : "=s"(hi));
  const uint32_t k1024 = static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(0x64006400u), 0xB1, 0xF, 0xF, true));
  const uint32_t k64 = static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(0x54005400u), 0xB1, 0xF, 0xF, true));
  return DqConst{lo, hi, k1024, k64};
}

__device__ __forceinline__ float h_lo(uint32_t p) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(p & 0xffffu)));
}
__device__ __forceinline__ float h_hi(uint32_t p) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(p >> 16)));
}

struct ColScale {
  float s, c1024, c72;  // s, -1032*s, -72*s
};

__device__ __forceinline__ ColScale col_scale(float s) {
  return ColScale{s, -1032.0f * s, -72.0f * s};
}

// One Marlin word -> bf16 pairs: (n0: k0k1, k8k9), (n1: k0k1, k8k9).
struct WordPairs {
  uint32_t n0_lo, n0_hi, n1_lo, n1_hi;
};

__device__ __forceinline__ WordPairs dequant_word(uint32_t x, const ColScale& a,
                                                  const ColScale& b, const DqConst& k) {
  const uint32_t p0 = and_or(x, k.m_lo, k.k1024);
  const uint32_t p1 = and_or(x, k.m_hi, k.k64);
  const uint32_t y = x >> 8;
  const uint32_t p2 = and_or(y, k.m_lo, k.k1024);
  const uint32_t p3 = and_or(y, k.m_hi, k.k64);
  WordPairs r;
  r.n0_lo = pack_bf16x2(__builtin_fmaf(h_lo(p0), a.s, a.c1024), __builtin_fmaf(h_hi(p0), a.s, a.c1024));
  r.n0_hi = pack_bf16x2(__builtin_fmaf(h_lo(p1), a.s, a.c72), __builtin_fmaf(h_hi(p1), a.s, a.c72));
  r.n1_lo = pack_bf16x2(__builtin_fmaf(h_lo(p2), b.s, b.c1024), __builtin_fmaf(h_hi(p2), b.s, b.c1024));
  r.n1_hi = pack_bf16x2(__builtin_fmaf(h_lo(p3), b.s, b.c72), __builtin_fmaf(h_hi(p3), b.s, b.c72));
  return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
  u32x4_t v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ floatx16_t mfma(bf16x8_t a, bf16x8_t b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// B fragments of one quant group (4 words of tile 2g+h) for X1, X2, Y1, Y2.
struct BFrags {
  bf16x8_t x1, x2, y1, y2;
};

__device__ __forceinline__ BFrags make_b(const uint32_t w[4], uint32_t scale_pair,
                                         const DqConst& k) {
  const ColScale a = col_scale(bf_lo(scale_pair));
  const ColScale b = col_scale(bf_hi(scale_pair));
  const WordPairs q0 = dequant_word(w[0], a, b, k);
  const WordPairs q1 = dequant_word(w[1], a, b, k);
  const WordPairs q2 = dequant_word(w[2], a, b, k);
  const WordPairs q3 = dequant_word(w[3], a, b, k);
  // Word jj holds k = 2jj + {0, 1} in its "lo" pair and 2jj + {8, 9} in its
  // "hi" pair, so the lo pairs of words 0..3 are k 0..7 and the hi pairs
  // k 8..15: fragment slots follow k in memory order, and the matching
  // activation fragments are plain 16-byte runs of the row.
  BFrags f;
  f.x1 = as_bf16x8(q0.n0_lo, q1.n0_lo, q2.n0_lo, q3.n0_lo);
  f.x2 = as_bf16x8(q0.n0_hi, q1.n0_hi, q2.n0_hi, q3.n0_hi);
  f.y1 = as_bf16x8(q0.n1_lo, q1.n1_lo, q2.n1_lo, q3.n1_lo);
  f.y2 = as_bf16x8(q0.n1_hi, q1.n1_hi, q2.n1_hi, q3.n1_hi);
  return f;
}

// Row of the 32x32 MFMA output held in accumulator element i by k-half h.
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

struct GemmArgs {
  const uint16_t* input;
  uint16_t* output;
  float* c_tmp;
  const uint32_t* qweight;
  const uint16_t* scales;
  int32_t* locks;
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* ntp;
  const float* topk_w;
  int sorted_len, bs, top_k, mul, size_m, size_n, size_k;
  int num_experts;  // expert ids outside [0, num_experts) are skipped
  int splits;       // decode: K split across `splits` workgroups (partial != nullptr)
  float* partial;   // non-null: fp32 partial sums [splits][size_m * top_k][size_n]
                    // instead of the bf16 output (finished by the consumer kernel)
  uint16_t* act;    // prefill, non-null: W13 + SwiGLU, act[sid][inter] instead of the output
  int inter;        // with act: gate columns [0, inter), up columns [inter, 2 inter)
};

__device__ __forceinline__ uint16_t epilogue_value(float acc, int sid, const GemmArgs& p) {
  uint16_t c = f2bf(acc);
  if (p.mul) c = f2bf(bf2f(c) * bf2f(f2bf(p.topk_w[sid])));
  return c;
}

// Raw buffer resources: base address in SGPRs, 32-bit per-lane offsets, a
// per-iteration scalar offset, and hardware range checking (reads at or past
// `bytes` return zero, which is how rows that are not routed here read zeros
// without a branch).
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
constexpr uint32_t kOutOfRange = 0x80000000u;  // voffset that fails every range check

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}
// Cache policy of a load: kCached for data other workgroups re-read (the
// activations), kStream (non-temporal) for bytes read exactly once per launch
// (the decode path's weights and scales), which then do not evict the rest.
constexpr int kCached = 0;
constexpr int kStream = 2;

template <int kPolicy = kCached>
__device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff),
                                              kPolicy);
}
template <int kPolicy = kCached>
__device__ __forceinline__ u32x4_t buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff),
                                               kPolicy);
}

// ---------------------------------------------------------------------------
// Decode kernel: one workgroup per (m-block, 64-column tile); WK waves split
// the K range and are reduced through LDS in a fixed wave order (bit-for-bit
// reproducible).  The block's rows (<= 32, one MFMA row block) occupy NI
// accumulator elements per lane (rows < bs).
//
// Weight traffic is shaped for the texture-address unit: per quant group a
// wave issues ONE 16-byte load per lane (lane L takes word row th = L%32 of
// k-tile 2g + L/32, i.e. both 512-byte tiles contiguously), then transposes
// through a per-wave LDS slot so that lane (c, h) reads its four fragment
// words (th = 4*(c%8) + jj, w = c/8) as one 16-byte LDS read.  Slot layout:
// word (th, w) of tile h at dword h*160 + w*32 + th (the 160 stride puts the
// two tiles in opposite bank halves: writes and reads are conflict-free).
// Each wave has two such slots, and a group's words are written one group
// ahead of their use, so the write-to-read LDS round trip overlaps the
// previous group's dequant instead of stalling its own.
// Lanes whose activation row is not routed here read zeros through an
// out-of-range buffer offset.  D groups per wave are in flight.
// ---------------------------------------------------------------------------
constexpr int kSlotDwords = 320;

struct GroupRegs {
  u32x4_t raw;  // 4 words (th, w = 0..3) of this lane's k-tile
  uint32_t sp;
  u32x4_t a;    // activations: row c % 16, k 16h + 8(c / 16) + 0..7
};

// kPair: W13 + SwiGLU.  The workgroup holds 2 WK waves: waves 0..WK-1 split K
// over a gate tile, waves WK..2WK-1 over the matching up tile (inter/64 tiles
// further), and the epilogue writes SwiGLU of the two bf16-rounded sums to
// p.act (p.output and p.partial are not used).
template <int WK, int NI, int D, bool kPair = false>
__global__ __launch_bounds__(64 * WK * (kPair ? 2 : 1), 4) void wna16_decode_kernel(GemmArgs p) {
  static_assert(D % 2 == 0, "the two transpose slots alternate with the ring position");
  constexpr int kWaves = WK * (kPair ? 2 : 1);
  __shared__ int s_sid[32];
  __shared__ float s_red[kWaves][2 * NI][64];
  __shared__ __align__(16) uint32_t s_w[kWaves][2][kSlotDwords];

  const int n_tiles = p.size_n >> 6;
  const int n_units = kPair ? (p.inter >> 6) : n_tiles;  // column units per K share
  const int split = blockIdx.x / n_units;
  const int mb = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int valid_limit = p.size_m * p.top_k;
  // The block's three index loads go out together, since none depends on
  // another: the routed total, the block's expert (mb < ceil(sorted_len / bs),
  // the grid's row count) and its rows' route ids.
  int sid = valid_limit;
  if (tid < p.bs && mb * p.bs + tid < p.sorted_len) sid = p.sorted_ids[mb * p.bs + tid];
  // readfirstlane: values the compiler cannot prove wave-uniform but that are
  // (block-level loads, wave index) go to SGPRs, so buffer descriptors and
  // scalar offsets built from them need no per-lane waterfall loops.
  const int expert = __builtin_amdgcn_readfirstlane(p.expert_ids[mb]);
  const int ntp = min(p.ntp[0], p.sorted_len);
  // one exit test over both values, so both loads are in flight together:
  // whole blocks only (mb < ntp / bs: rows stay inside sorted_len), local
  // experts only
  if (ntp < (mb + 1) * p.bs || expert < 0 || expert >= p.num_experts) return;

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave % WK;    // this wave's K share
  const int half = wave / WK;  // with kPair: 0 gate tile, 1 up tile
  const int nt = blockIdx.x % n_units + (kPair ? half * (p.inter >> 6) : 0);
  if (tid < 32) s_sid[tid] = sid;
  __syncthreads();

  const int c = lane & 31, h = lane >> 5;
  const int K = p.size_k, N = p.size_n;
  const int groups = K >> 5;
  // this workgroup's share of the K groups, then this wave's share of that
  const int gs0 = (groups * split) / p.splits, gs1 = (groups * (split + 1)) / p.splits;
  const int g0 = gs0 + ((gs1 - gs0) * kw) / WK, g1 = gs0 + ((gs1 - gs0) * (kw + 1)) / WK;

  const uint32_t expert_bytes = static_cast<uint32_t>(N) * static_cast<uint32_t>(K) / 2u;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(
      p.qweight + static_cast<long long>(expert) * (expert_bytes / 4u), expert_bytes);
  const uint32_t tile_row_bytes = static_cast<uint32_t>(n_tiles) * 512u;
  const uint32_t w_voff = static_cast<uint32_t>(h) * tile_row_bytes +
                          static_cast<uint32_t>(nt) * 512u + static_cast<uint32_t>(c) * 16u;
  const uint32_t w_step = 2u * tile_row_bytes;  // bytes per quant group
  const uint32_t scale_bytes = static_cast<uint32_t>(groups) * static_cast<uint32_t>(N) * 2u;
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(
      p.scales + static_cast<long long>(expert) * groups * N, scale_bytes);
  const uint32_t s_voff = (static_cast<uint32_t>(nt) * 64u + 8u * (c & 7) + 2u * (c >> 3)) * 2u;
  const uint32_t s_step = static_cast<uint32_t>(N) * 2u;
  // Row folding: a block has at most 16 rows, so MFMA rows 16..31 are free.
  // Lane (c, h) loads ONE 16-byte run per group: row c % 16, k 16h + 8(c/16)
  // + 0..7.  Against the k 0..7 weight fragments (x1, y1) rows 0..15 are the
  // real products; against the k 8..15 fragments (x2, y2) rows 16..31 are
  // (rows 0..15 shifted by 16).  Separate lo / hi accumulators keep the
  // unrelated halves apart, and the row's sum is lo[i] + hi[i + 8]: the same
  // lane, 8 elements further.  One activation load per group instead of two.
  const int my_sid = s_sid[c & 15];
  const __amdgpu_buffer_rsrc_t ar =
      make_rsrc(p.input, static_cast<uint32_t>(p.size_m) * static_cast<uint32_t>(K) * 2u);
  const uint32_t a_voff =
      static_cast<unsigned>(my_sid) < static_cast<unsigned>(valid_limit)
          ? (static_cast<uint32_t>(my_sid / p.top_k) * static_cast<uint32_t>(K) + 16u * h +
             8u * static_cast<uint32_t>(c >> 4)) * 2u
          : kOutOfRange;

  uint32_t* slot_w0 = &s_w[wave][0][h * 160 + c];          // this lane's write column
  uint32_t* slot_w1 = &s_w[wave][1][h * 160 + c];
  const uint32_t* slot_r0 = &s_w[wave][0][h * 160 + 4 * c];  // this lane's 16-byte read
  const uint32_t* slot_r1 = &s_w[wave][1][h * 160 + 4 * c];

  auto load_group = [&](GroupRegs& r, int g) {
    g = min(max(g, 0), groups - 1);  // every scalar offset stays inside the expert
    r.raw = buf_load_b128<kStream>(wr, w_voff, static_cast<uint32_t>(g) * w_step);
    r.sp = buf_load_b32<kStream>(sr, s_voff, static_cast<uint32_t>(g) * s_step);
    // rows not routed here have an out-of-range offset and read zeros; no
    // branch, so the loads stay in flight across groups
    r.a = buf_load_b128(ar, a_voff, static_cast<uint32_t>(g) * 64u);
  };

  const DqConst dq = dq_consts();
  floatx16_t accx_lo = {}, accx_hi = {}, accy_lo = {}, accy_hi = {};
  GroupRegs slot[D];
#pragma unroll
  for (int q = 0; q < D; ++q) {
    load_group(slot[q], g0 + q < g1 ? g0 + q : g1 - 1);
    // keep the issue order slot by slot (weights, scale, activations), the
    // order the main loop refills in, so that each group's wait counts only
    // its own three loads
    __builtin_amdgcn_sched_barrier(0);
  }

  // transpose a group's tile words into fragment order through slot `par`
  auto write_tr = [&](const GroupRegs& r, int par) {
    uint32_t* sw = par ? slot_w1 : slot_w0;
    sw[0] = r.raw[0];
    sw[32] = r.raw[1];
    sw[64] = r.raw[2];
    sw[96] = r.raw[3];
  };
  auto compute_group = [&](const GroupRegs& r, int par) {
    const u32x4_t fw = *reinterpret_cast<const u32x4_t*>(par ? slot_r1 : slot_r0);
    const uint32_t w4[4] = {fw[0], fw[1], fw[2], fw[3]};
    const BFrags b = make_b(w4, r.sp, dq);
    const bf16x8_t A = __builtin_bit_cast(bf16x8_t, r.a);
    accx_lo = mfma(A, b.x1, accx_lo);
    accx_hi = mfma(A, b.x2, accx_hi);
    accy_lo = mfma(A, b.y1, accy_lo);
    accy_hi = mfma(A, b.y2, accy_hi);
  };

  // Main loop over whole rounds of D groups: no branch inside, so the loads
  // of the next round stay in flight while this round computes.  The slot a
  // group came from is refilled with the group D ahead (clamped to the last
  // group of the slice, fetched again and never used).  The scheduling
  // barrier pins each refill right after its slot's compute: left free, the
  // scheduler sinks all refills to the end of the unrolled round, and the
  // next round then opens with vmcnt(0), waiting out a full memory latency.
  // Pinned, group q waits only for its own loads while the D - 1 later
  // groups' loads stay in flight (C3 W13 117.5 -> 113.3 us).  Step q first
  // writes the transpose of the next group (ring slot q + 1, or slot 0, which
  // step 0 refilled with the group D ahead), into the other LDS slot: a slot
  // is rewritten only after the wave's read of it, and a wave's LDS
  // operations complete in order.
  const int rounds = (g1 - g0) / D;
  int g = g0;
  write_tr(slot[0], 0);
  for (int r = 0; r < rounds; ++r, g += D) {
#pragma unroll
    for (int q = 0; q < D; ++q) {
      write_tr(slot[(q + 1) % D], (q + 1) & 1);
      compute_group(slot[q], q & 1);
      load_group(slot[q], min(g + q + D, g1 - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int q = 0; q < D - 1; ++q) {
    if (g + q < g1) {
      if (q + 1 < D - 1 && g + q + 1 < g1) write_tr(slot[q + 1], (q + 1) & 1);
      compute_group(slot[q], q & 1);
    }
  }

  // Deterministic reduction over the WK waves (fixed order 0..WK-1); only the
  // NI accumulator elements that hold rows < bs are exchanged, each the sum
  // of its k-lo part (rows 0..15) and k-hi part (folded to rows 16..31).
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    s_red[wave][i][lane] = accx_lo[i] + accx_hi[i + 8];
    s_red[wave][NI + i][lane] = accy_lo[i] + accy_hi[i + 8];
  }
  __syncthreads();

  if constexpr (kPair) {
    // the same (row, column) of the gate and the up tile: SwiGLU of the two sums
    const int col0 = (blockIdx.x % n_units) * 64 + (c >> 3) * 16 + (c & 7);
    for (int j = wave; j < 2 * NI; j += kWaves) {
      float sg = 0.0f, su = 0.0f;
#pragma unroll
      for (int w = 0; w < WK; ++w) {
        sg += s_red[w][j][lane];
        su += s_red[WK + w][j][lane];
      }
      const int row = acc_row(j < NI ? j : j - NI, h);
      const int col = (j < NI) ? col0 : col0 + 8;
      if (row < p.bs) {
        const int sid = s_sid[row];
        if (static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit))
          p.act[static_cast<long long>(sid) * p.inter + col] =
              swiglu_one(bf2f(f2bf(sg)), bf2f(f2bf(su)));
      }
    }
    return;
  }
  const int n0 = nt * 64 + (c >> 3) * 16 + (c & 7);
  for (int j = wave; j < 2 * NI; j += WK) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < WK; ++w) s += s_red[w][j][lane];
    const int row = acc_row(j < NI ? j : j - NI, h);
    const int n = (j < NI) ? n0 : n0 + 8;
    if (row < p.bs) {
      const int sid = s_sid[row];
      if (static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit)) {
        if (p.partial)
          p.partial[(static_cast<long long>(split) * valid_limit + sid) * N + n] = s;
        else
          p.output[static_cast<long long>(sid) * N + n] = epilogue_value(s, sid, p);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode kernel on v_mfma_f32_16x16x32_bf16, used at WK = 4 (C3's W13 pair,
// the paired and plain W13 GEMMs alike, and its W2).  A block's 16 rows are the
// MFMA's 16 rows, so the accumulators are 16 VGPRs per lane instead of the
// 32-row form's 64 (whose rows 16..31 only fold k): 80 VGPRs, six waves per
// SIMD instead of four, and three 8-wave W13 workgroups per CU instead of two.
// A wave's 64 columns are four 16-column MFMA tiles.  Lane (n16 = cc + 8 a2,
// kb = 2 kt + hf) takes the Marlin column pairs (w = 2 a2, cc) and
// (w = 2 a2 + 1, cc) -- real columns 32 a2 + 8 j + cc for MFMA j -- and words
// jj = 2 hf, 2 hf + 1 of k-tile kt, read from the same transpose slots as the
// 32-row kernel with one 8-byte read per pair; its B fragments then hold
// k 16 kt + 4 hf + {0..3, 8..11} (a word's nibbles are k 2jj + {0, 1, 8, 9}).
// The activation fragment takes the same k set: each lane loads 16 bytes
// (k 16 kt + 8 hf + 0..7) and a permlane16 swap exchanges the middle 8 bytes
// with the lanes of the other k half.  The dequant is the 32-row kernel's; a
// lane now scales four columns instead of two, and the two k halves' lanes
// take one 8-byte scale load.  C3's W13 pair: 122.5 -> 119.2 us, W2 at WK = 4
// instead of 2: 65.4 -> 64.0 us (three interleaved rounds, one box).  The swap's
// output goes into the fragment with no per-lane select (both k halves find the
// swapped bytes in the same registers): 121.9 -> 117.0 us and 64.6 -> 62.9 us.
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;

__device__ __forceinline__ floatx4_t mfma16(bf16x8_t a, bf16x8_t b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct GroupRegs16 {
  u32x4_t raw;
  uint32_t sp0, sp1;  // scales: pair A (n0, n1), pair B (n0, n1)
  u32x4_t a;
};

template <int WK, int D, bool kPair = false>
__global__ __launch_bounds__(64 * WK * (kPair ? 2 : 1), 6) void wna16_decode16_kernel(GemmArgs p) {
  static_assert(D % 2 == 0, "the two transpose slots alternate with the ring position");
  constexpr int kWaves = WK * (kPair ? 2 : 1);
  __shared__ int s_sid[32];
  __shared__ float s_red[kWaves][16][64];
  __shared__ __align__(16) uint32_t s_w[kWaves][2][kSlotDwords];

  const int n_tiles = p.size_n >> 6;
  const int n_units = kPair ? (p.inter >> 6) : n_tiles;
  const int split = blockIdx.x / n_units;
  const int mb = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int valid_limit = p.size_m * p.top_k;
  int sid = valid_limit;
  if (tid < p.bs && mb * p.bs + tid < p.sorted_len) sid = p.sorted_ids[mb * p.bs + tid];
  const int expert = __builtin_amdgcn_readfirstlane(p.expert_ids[mb]);
  const int ntp = min(p.ntp[0], p.sorted_len);
  if (ntp < (mb + 1) * p.bs || expert < 0 || expert >= p.num_experts) return;

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave % WK;
  const int half = wave / WK;
  const int nt = blockIdx.x % n_units + (kPair ? half * (p.inter >> 6) : 0);
  if (tid < 32) s_sid[tid] = sid;
  __syncthreads();

  // loader view (as the 32x32 kernel): lane L holds word row th = L%32 of tile L/32
  const int c = lane & 31, h = lane >> 5;
  // MFMA view
  const int n16 = lane & 15, kb = lane >> 4;
  const int cc = n16 & 7, a2 = n16 >> 3;  // column pair index and pair-of-pairs
  const int kt = kb >> 1, hf = kb & 1;    // k-tile within the group, k half
  const int K = p.size_k, N = p.size_n;
  const int groups = K >> 5;
  const int gs0 = (groups * split) / p.splits, gs1 = (groups * (split + 1)) / p.splits;
  const int g0 = gs0 + ((gs1 - gs0) * kw) / WK, g1 = gs0 + ((gs1 - gs0) * (kw + 1)) / WK;

  const uint32_t expert_bytes = static_cast<uint32_t>(N) * static_cast<uint32_t>(K) / 2u;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(
      p.qweight + static_cast<long long>(expert) * (expert_bytes / 4u), expert_bytes);
  const uint32_t tile_row_bytes = static_cast<uint32_t>(n_tiles) * 512u;
  const uint32_t w_voff = static_cast<uint32_t>(h) * tile_row_bytes +
                          static_cast<uint32_t>(nt) * 512u + static_cast<uint32_t>(c) * 16u;
  const uint32_t w_step = 2u * tile_row_bytes;
  const uint32_t scale_bytes = static_cast<uint32_t>(groups) * static_cast<uint32_t>(N) * 2u;
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(
      p.scales + static_cast<long long>(expert) * groups * N, scale_bytes);
  // pairs (2a2, cc) and (2a2 + 1, cc): bf16 scales 8cc + 4a2 + 0..3 of the tile
  const uint32_t s_voff = (static_cast<uint32_t>(nt) * 64u + 8u * cc + 4u * a2) * 2u;
  const uint32_t s_step = static_cast<uint32_t>(N) * 2u;
  // activations: row n16, bytes 32 kt + 16 hf .. +15 of the group's 64
  const int my_sid = s_sid[n16];
  const __amdgpu_buffer_rsrc_t ar =
      make_rsrc(p.input, static_cast<uint32_t>(p.size_m) * static_cast<uint32_t>(K) * 2u);
  const uint32_t a_voff =
      static_cast<unsigned>(my_sid) < static_cast<unsigned>(valid_limit)
          ? (static_cast<uint32_t>(my_sid / p.top_k) * static_cast<uint32_t>(K)) * 2u +
                32u * kt + 16u * hf
          : kOutOfRange;

  uint32_t* slot_w0 = &s_w[wave][0][h * 160 + c];
  uint32_t* slot_w1 = &s_w[wave][1][h * 160 + c];
  const int rd = kt * 160 + 64 * a2 + 4 * cc + 2 * hf;  // pair A's two words; pair B's +32
  const uint32_t* slot_r0 = &s_w[wave][0][rd];
  const uint32_t* slot_r1 = &s_w[wave][1][rd];

  auto load_group = [&](GroupRegs16& r, int g) {
    g = min(max(g, 0), groups - 1);
    r.raw = buf_load_b128<kStream>(wr, w_voff, static_cast<uint32_t>(g) * w_step);
    const auto sp = __builtin_amdgcn_raw_buffer_load_b64(sr, static_cast<int>(s_voff),
                                                         static_cast<int>(g * s_step), kStream);
    r.sp0 = sp[0];
    r.sp1 = sp[1];
    r.a = buf_load_b128(ar, a_voff, static_cast<uint32_t>(g) * 64u);
  };

  const DqConst dq = dq_consts();
  floatx4_t acc[4] = {};
  GroupRegs16 slot[D];
#pragma unroll
  for (int q = 0; q < D; ++q) {
    load_group(slot[q], g0 + q < g1 ? g0 + q : g1 - 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  auto write_tr = [&](const GroupRegs16& r, int par) {
    uint32_t* sw = par ? slot_w1 : slot_w0;
    sw[0] = r.raw[0];
    sw[32] = r.raw[1];
    sw[64] = r.raw[2];
    sw[96] = r.raw[3];
  };
  auto compute_group = [&](const GroupRegs16& r, int par) {
    const uint32_t* sr_ = par ? slot_r1 : slot_r0;
    const uint32_t wA0 = sr_[0], wA1 = sr_[1], wB0 = sr_[32], wB1 = sr_[33];
    const ColScale sA0 = col_scale(bf_lo(r.sp0)), sA1 = col_scale(bf_hi(r.sp0));
    const ColScale sB0 = col_scale(bf_lo(r.sp1)), sB1 = col_scale(bf_hi(r.sp1));
    const WordPairs qa0 = dequant_word(wA0, sA0, sA1, dq);
    const WordPairs qa1 = dequant_word(wA1, sA0, sA1, dq);
    const WordPairs qb0 = dequant_word(wB0, sB0, sB1, dq);
    const WordPairs qb1 = dequant_word(wB1, sB0, sB1, dq);
    // activations: swap the middle 8 bytes with the other k half's lanes (the odd
    // 16-lane rows of the first operand with the even rows of the second), after
    // which both halves find their fragment in the same registers
    const auto s0 = __builtin_amdgcn_permlane16_swap(r.a[0], r.a[2], false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(r.a[1], r.a[3], false, false);
    const bf16x8_t A = as_bf16x8(s0[0], s1[0], s0[1], s1[1]);
    acc[0] = mfma16(A, as_bf16x8(qa0.n0_lo, qa1.n0_lo, qa0.n0_hi, qa1.n0_hi), acc[0]);
    acc[1] = mfma16(A, as_bf16x8(qa0.n1_lo, qa1.n1_lo, qa0.n1_hi, qa1.n1_hi), acc[1]);
    acc[2] = mfma16(A, as_bf16x8(qb0.n0_lo, qb1.n0_lo, qb0.n0_hi, qb1.n0_hi), acc[2]);
    acc[3] = mfma16(A, as_bf16x8(qb0.n1_lo, qb1.n1_lo, qb0.n1_hi, qb1.n1_hi), acc[3]);
  };

  const int rounds = (g1 - g0) / D;
  int g = g0;
  write_tr(slot[0], 0);
  for (int r = 0; r < rounds; ++r, g += D) {
#pragma unroll
    for (int q = 0; q < D; ++q) {
      write_tr(slot[(q + 1) % D], (q + 1) & 1);
      compute_group(slot[q], q & 1);
      load_group(slot[q], min(g + q + D, g1 - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int q = 0; q < D - 1; ++q) {
    if (g + q < g1) {
      if (q + 1 < D - 1 && g + q + 1 < g1) write_tr(slot[q + 1], (q + 1) & 1);
      compute_group(slot[q], q & 1);
    }
  }

  // element e = 4j + i of a lane: row 4 kb + i, column 32 a2 + 8 j + cc
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[wave][4 * j + i][lane] = acc[j][i];
  __syncthreads();

  if constexpr (kPair) {
    const int colb = (blockIdx.x % n_units) * 64 + 32 * a2 + cc;
    for (int e = wave; e < 16; e += kWaves) {
      float sg = 0.0f, su = 0.0f;
#pragma unroll
      for (int w = 0; w < WK; ++w) {
        sg += s_red[w][e][lane];
        su += s_red[WK + w][e][lane];
      }
      const int row = 4 * kb + (e & 3);
      const int col = colb + 8 * (e >> 2);
      if (row < p.bs) {
        const int rsid = s_sid[row];
        if (static_cast<unsigned>(rsid) < static_cast<unsigned>(valid_limit))
          p.act[static_cast<long long>(rsid) * p.inter + col] =
              swiglu_one(bf2f(f2bf(sg)), bf2f(f2bf(su)));
      }
    }
    return;
  }
  const int colb = nt * 64 + 32 * a2 + cc;
  for (int e = wave; e < 16; e += WK) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < WK; ++w) s += s_red[w][e][lane];
    const int row = 4 * kb + (e & 3);
    const int n = colb + 8 * (e >> 2);
    if (row < p.bs) {
      const int rsid = s_sid[row];
      if (static_cast<unsigned>(rsid) < static_cast<unsigned>(valid_limit)) {
        if (p.partial)
          p.partial[(static_cast<long long>(split) * valid_limit + rsid) * N + n] = s;
        else
          p.output[static_cast<long long>(rsid) * N + n] = epilogue_value(s, rsid, p);
      }
    }
  }
}

constexpr int kDecodeDepth = 4;

// WK = 4 runs the 16x16x32 kernel, the other share counts the 32-row one
// (at 8 and 16 waves per workgroup the 16x16x32 form gains no occupancy and
// its extra scale work cost C1/C2 2-4%).
template <int WK>
void launch_decode(const GemmArgs& args, int max_m_blocks, hipStream_t stream) {
  const dim3 grid(args.size_n / 64 * args.splits, max_m_blocks);
  if constexpr (WK == 4) {
    hipLaunchKernelGGL((wna16_decode16_kernel<WK, kDecodeDepth>), grid, dim3(64 * WK), 0, stream,
                       args);
  } else {
    if (args.bs <= 8)
      hipLaunchKernelGGL((wna16_decode_kernel<WK, 4, kDecodeDepth>), grid, dim3(64 * WK), 0,
                         stream, args);
    else
      hipLaunchKernelGGL((wna16_decode_kernel<WK, 8, kDecodeDepth>), grid, dim3(64 * WK), 0,
                         stream, args);
  }
}

template <int WK>
void launch_decode_pair(const GemmArgs& args, int max_m_blocks, hipStream_t stream) {
  const dim3 grid(args.inter / 64, max_m_blocks);
  if constexpr (WK == 4) {
    hipLaunchKernelGGL((wna16_decode16_kernel<WK, kDecodeDepth, true>), grid, dim3(128 * WK), 0,
                       stream, args);
  } else {
    if (args.bs <= 8)
      hipLaunchKernelGGL((wna16_decode_kernel<WK, 4, kDecodeDepth, true>), grid, dim3(128 * WK),
                         0, stream, args);
    else
      hipLaunchKernelGGL((wna16_decode_kernel<WK, 8, kDecodeDepth, true>), grid, dim3(128 * WK),
                         0, stream, args);
  }
}

// ---------------------------------------------------------------------------
// Prefill kernel: one workgroup per (leader m-block, 4 column tiles); the
// leader takes up to R/bs consecutive m-blocks of the same expert (an R-row
// tile, R = 128, or 64 where experts hold few rows), 4 waves each own one
// 64-column tile.
//
// Per 64-wide K chunk (two quant groups):
//   * activations: 128 rows x 64 k (16 KB) staged in double-buffered LDS
//     (rows padded to 72 bf16 against bank conflicts), loaded by all 256
//     threads with 16-byte buffer loads two chunks ahead of use;
//   * weights: one 16-byte load per lane per group (the decode kernel's
//     pattern), transposed through a per-wave LDS slot, dequantised in
//     registers; two chunks in flight;
//   * 16 MFMA 32x32x16 per group per wave (4 row blocks x n0/n1 x 2 k-halves).
// The loop is unrolled by two with named ping-pong buffers, so no register
// copies are needed to rotate the prefetch; activation loads are issued
// before weight loads so that waiting for the former leaves the latter in
// flight (vector-memory counters retire in order).
// ---------------------------------------------------------------------------
constexpr int kPfChunk = 64;                 // k per LDS stage (2 quant groups)
constexpr int kPfLdsStride = kPfChunk + 8;   // bf16 per LDS row (padding vs bank conflicts)
// bf16 elements of the LDS area of an R-row tile: the two activation stages,
// or the epilogue's 64-row staging ([64][264] bf16, or [2][64][65] words)
constexpr int pf_lds_elems(int R) {
  return 2 * R * kPfLdsStride > 64 * 264 ? 2 * R * kPfLdsStride : 64 * 264;
}

struct PfB {
  u32x4_t w[2];   // per group: the 4 words (th, w = 0..3) of this lane's k-tile
  uint32_t s[2];  // per group: this lane's two column scales
};

// Main loop and epilogue of one wave for a tile with RB routed 32-row blocks
// (RB = 0: a wave past the last column tile, which only helps stage the
// activations).  A compile-time RB keeps every loop body branch-free and
// allocates only the accumulators in use.
template <int RB, int R>
__device__ __forceinline__ void prefill_tile(const GemmArgs& p, uint16_t* s_a, uint32_t* s_w_wave,
                                             const int* s_sid, const float* s_tw, int expert,
                                             int nt, int tx) {
  constexpr int kStage = R * kPfLdsStride;  // bf16 per activation stage
  constexpr int kPieces = R / 32;           // 16-byte activation pieces per thread per chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int c = lane & 31, h = lane >> 5;
  const int K = p.size_k, N = p.size_n;
  const int n_tiles = N >> 6;
  const int groups = K >> 5;
  const int chunks = K / kPfChunk;
  const int valid_limit = p.size_m * p.top_k;
  const int ntc = RB > 0 ? nt : 0;
  const uint32_t expert_bytes = static_cast<uint32_t>(N) * static_cast<uint32_t>(K) / 2u;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(
      p.qweight + static_cast<long long>(expert) * (expert_bytes / 4u), expert_bytes);
  const uint32_t tile_row_bytes = static_cast<uint32_t>(n_tiles) * 512u;
  const uint32_t w_voff = static_cast<uint32_t>(h) * tile_row_bytes +
                          static_cast<uint32_t>(ntc) * 512u + static_cast<uint32_t>(c) * 16u;
  const uint32_t w_step = 2u * tile_row_bytes;  // bytes per quant group
  const uint32_t scale_bytes = static_cast<uint32_t>(groups) * static_cast<uint32_t>(N) * 2u;
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(
      p.scales + static_cast<long long>(expert) * groups * N, scale_bytes);
  const uint32_t s_voff = (static_cast<uint32_t>(ntc) * 64u + 8u * (c & 7) + 2u * (c >> 3)) * 2u;
  const uint32_t s_step = static_cast<uint32_t>(N) * 2u;
  const __amdgpu_buffer_rsrc_t ar =
      make_rsrc(p.input, static_cast<uint32_t>(p.size_m) * static_cast<uint32_t>(K) * 2u);

  uint32_t* slot_w = s_w_wave + h * 160 + c;          // this lane's transpose write column
  const uint32_t* slot_r = s_w_wave + h * 160 + 4 * c;  // this lane's 16-byte read

  auto load_b = [&](PfB& b, int chunk) {
    if constexpr (RB > 0) {
      const uint32_t ch = static_cast<uint32_t>(min(chunk, chunks - 1));  // past the end: unused
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const uint32_t g = 2u * ch + static_cast<uint32_t>(gg);
        b.w[gg] = buf_load_b128(wr, w_voff, g * w_step);
        b.s[gg] = buf_load_b32(sr, s_voff, g * s_step);
      }
    }
  };

  // Activation staging: R rows x 64 k = 8 R 16-byte pieces, R / 32 per thread;
  // rows not routed here read zeros (out-of-range buffer offset).  A thread's
  // piece i lies in 32-row block i, so a tile with RB < R / 32 routed blocks
  // stages only its first RB blocks (the MFMAs read no other row); a wave past
  // the last column tile (RB = 0) stages all of them, which covers whatever
  // the workgroup's other waves need.
  constexpr int kStaged = RB > 0 && RB < kPieces ? RB : kPieces;
  uint32_t a_voff[kStaged];
#pragma unroll
  for (int i = 0; i < kStaged; ++i) {
    const int piece = tid + 256 * i;
    const int r = piece >> 3, q = piece & 7;
    const int sid = s_sid[r];
    a_voff[i] = static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit)
                    ? (static_cast<uint32_t>(sid / p.top_k) * static_cast<uint32_t>(K) + 8u * q) * 2u
                    : kOutOfRange;
  }
  // A chunk index past the end reads zeros (every lane out of range).
  auto load_a = [&](u32x4_t (&st)[kStaged], int chunk) {
    const uint32_t past = chunk < chunks ? 0u : kOutOfRange;
    const uint32_t ch = static_cast<uint32_t>(min(chunk, chunks - 1));
#pragma unroll
    for (int i = 0; i < kStaged; ++i)
      st[i] = buf_load_b128(ar, a_voff[i] | past, ch * (kPfChunk * 2u));
  };
  auto store_a = [&](const u32x4_t (&st)[kStaged], int buf) {
#pragma unroll
    for (int i = 0; i < kStaged; ++i) {
      const int piece = tid + 256 * i;
      const int r = piece >> 3, q = piece & 7;
      *reinterpret_cast<u32x4_t*>(&s_a[buf * kStage + r * kPfLdsStride + 8 * q]) = st[i];
    }
  };

  constexpr int NACC = RB > 0 ? RB : 1;
  floatx16_t accx[NACC], accy[NACC];
#pragma unroll
  for (int rb = 0; rb < NACC; ++rb) {
    accx[rb] = floatx16_t{};
    accy[rb] = floatx16_t{};
  }
  const DqConst dq = dq_consts();

  auto compute = [&](const PfB& b, int buf) {
    if constexpr (RB > 0) {
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        // transpose the tile words into fragment order through this wave's slot
        slot_w[0] = b.w[gg][0];
        slot_w[32] = b.w[gg][1];
        slot_w[64] = b.w[gg][2];
        slot_w[96] = b.w[gg][3];
        const u32x4_t fw = *reinterpret_cast<const u32x4_t*>(slot_r);
        const uint32_t w4[4] = {fw[0], fw[1], fw[2], fw[3]};
        const BFrags f = make_b(w4, b.s[gg], dq);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const uint16_t* ap = &s_a[buf * kStage + (32 * rb + c) * kPfLdsStride + 32 * gg + 16 * h];
          const bf16x8_t A1 = *reinterpret_cast<const bf16x8_t*>(ap);
          const bf16x8_t A2 = *reinterpret_cast<const bf16x8_t*>(ap + 8);
          accx[rb] = mfma(A1, f.x1, accx[rb]);
          accx[rb] = mfma(A2, f.x2, accx[rb]);
          accy[rb] = mfma(A1, f.y1, accy[rb]);
          accy[rb] = mfma(A2, f.y2, accy[rb]);
        }
      }
    }
  };

  PfB b_even, b_odd;
  u32x4_t st_even[kStaged], st_odd[kStaged];
  load_a(st_even, 0);
  load_b(b_even, 0);
  load_a(st_odd, 1);
  load_b(b_odd, 1);
  store_a(st_even, 0);
  __syncthreads();
  // Invariant at the top of each pair: s_a[0] holds chunk ch, st_odd holds
  // (or is loading) chunk ch + 1, b_even / b_odd hold chunks ch / ch + 1.
  // One exit only and no tail copy of the loop body, so the accumulators
  // keep their registers.  With an odd chunk count the last pair's second
  // chunk is past the end: its activations are zeros, and adding +0 to an
  // accumulator that started at +0 changes nothing.
  const int pairs = (chunks + 1) >> 1;
  for (int pr = 0; pr < pairs; ++pr) {
    const int ch = 2 * pr;
    load_a(st_even, ch + 2);
    compute(b_even, 0);
    load_b(b_even, ch + 2);
    // s_a[1] was last read in the previous pair, before the barrier that ended it
    store_a(st_odd, 1);
    __syncthreads();
    load_a(st_odd, ch + 3);
    compute(b_odd, 1);
    load_b(b_odd, ch + 3);
    // every wave finished reading s_a[0] (chunk ch) before the barrier above;
    // past the last chunk this stages a clamped copy nobody reads
    store_a(st_even, 0);
    __syncthreads();
  }

  if (p.act != nullptr) {
    // W13 + SwiGLU in two row halves (rows 64 ph .. 64 ph + 63, the 32-row
    // blocks 2 ph and 2 ph + 1): the gate and up waves of both tile pairs put
    // their bf16 values into the activation stages (free since the loop's last
    // barrier) as [pair][64 rows][65] words, gate in the low half and up in the
    // high half; then each thread finishes half a row of one pair (32 columns,
    // four 16-byte stores).  Every wave passes the same four barriers whatever
    // its routed-block count.
    constexpr int kXStride = 65;  // words per row (odd: the two k-halves' rows use other banks)
    uint16_t* x16 = reinterpret_cast<uint16_t*>(s_a);
    const uint32_t* x32 = reinterpret_cast<const uint32_t*>(s_a);
    const int wave = threadIdx.x >> 6;
    const int g0 = tx * 2;  // first gate tile of this workgroup
    const int gate_tiles = p.inter >> 6;
#pragma unroll
    for (int ph = 0; ph < R / 64; ++ph) {
      if constexpr (RB > 0) {
        const int pair = wave & 1, half = wave >> 1;  // half 0: gate, 1: up
        const int col = (c >> 3) * 16 + (c & 7);
#pragma unroll
        for (int rbl = 0; rbl < 2; ++rbl) {
          const int rb = 2 * ph + rbl;
          if (rb < RB) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int row = 32 * rbl + acc_row(i, h);
              uint16_t* x = x16 + ((pair * 64 + row) * kXStride + col) * 2 + half;
              x[0] = f2bf(accx[rb < NACC ? rb : 0][i]);
              x[16] = f2bf(accy[rb < NACC ? rb : 0][i]);  // column col + 8
            }
          }
        }
      }
      __syncthreads();
      const int pair_t = threadIdx.x >> 7, r = (threadIdx.x >> 1) & 63, part = threadIdx.x & 1;
      const int sid = s_sid[64 * ph + r];
      if (g0 + pair_t < gate_tiles &&
          static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit)) {
        const uint32_t* src = x32 + (pair_t * 64 + r) * kXStride + 32 * part;
        uint16_t* dst =
            p.act + static_cast<long long>(sid) * p.inter + (g0 + pair_t) * 64 + 32 * part;
#pragma unroll 1
        for (int q = 0; q < 4; ++q) {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t v0 = src[8 * q + 2 * e], v1 = src[8 * q + 2 * e + 1];
            const uint16_t lo = swiglu_one(bf2f(static_cast<uint16_t>(v0 & 0xffffu)),
                                           bf2f(static_cast<uint16_t>(v0 >> 16)));
            const uint16_t hi = swiglu_one(bf2f(static_cast<uint16_t>(v1 & 0xffffu)),
                                           bf2f(static_cast<uint16_t>(v1 >> 16)));
            w[e] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
          }
          *reinterpret_cast<uint4*>(dst + 8 * q) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      __syncthreads();  // the next half reuses the stages
    }
    return;
  }
  // bf16 output (times the row's bf16 top-k weight with mul), in two row
  // halves: the waves put their values for rows 64 ph .. 64 ph + 63 into the
  // activation stages as [64 rows][264] bf16 (the four tiles side by side),
  // then each thread stores one tile's 64 columns of a row with 16-byte stores.
  constexpr int kOStride = 264;  // bf16 per row: 256 + 8, rows start on other banks
  uint16_t* xo = reinterpret_cast<uint16_t*>(s_a);
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int ph = 0; ph < R / 64; ++ph) {
    if constexpr (RB > 0) {
      const int col = wave * 64 + (c >> 3) * 16 + (c & 7);
#pragma unroll
      for (int rbl = 0; rbl < 2; ++rbl) {
        const int rb = 2 * ph + rbl;
        if (rb < RB) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int row = 32 * rbl + acc_row(i, h);
            uint16_t vx = f2bf(accx[rb < NACC ? rb : 0][i]);
            uint16_t vy = f2bf(accy[rb < NACC ? rb : 0][i]);
            if (p.mul) {
              const float w = s_tw[64 * ph + row];
              vx = f2bf(bf2f(vx) * w);
              vy = f2bf(bf2f(vy) * w);
            }
            xo[row * kOStride + col] = vx;
            xo[row * kOStride + col + 8] = vy;
          }
        }
      }
    }
    __syncthreads();
    const int r = threadIdx.x >> 2, t4 = threadIdx.x & 3;
    const int sid = s_sid[64 * ph + r];
    const int nt_t = tx * 4 + t4;
    if (nt_t < (N >> 6) && static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit)) {
      const uint4* src = reinterpret_cast<const uint4*>(xo + r * kOStride + t4 * 64);
      uint4* dst = reinterpret_cast<uint4*>(p.output + static_cast<long long>(sid) * N + nt_t * 64);
#pragma unroll
      for (int q = 0; q < 8; ++q) dst[q] = src[q];
    }
    __syncthreads();  // the next half reuses the stages
  }
}

// The tiles of one launch: every m-block whose position in its expert's run of
// blocks is a multiple of the blocks-per-tile count starts a tile.  Workgroup
// row y takes the y-th such block in block order, found by a ballot scan of
// the block experts, so the grid holds the tiles first and the rows past the
// last tile at its end.  (Rows indexed by m-block instead leave an idle
// workgroup after every leader in dispatch order, and the round-robin spread
// over shader engines then puts all the work on half of them.)
constexpr int kPfScanSlab = 1024;  // block experts staged in LDS per scan pass

// One workgroup's tile of a problem: column group tx, tile ty.  Up to
// kPfScanSlab blocks, the tiles that hold all R / bs of their blocks come first
// and the shorter last tiles of the experts after them (each group in block
// order), so the short tiles fill the end of the launch; past that many
// blocks, block order.
template <int R>
__device__ __forceinline__ void prefill_block(const GemmArgs& p, int tx, int ty) {
  __shared__ __align__(16) uint16_t s_a[pf_lds_elems(R)];
  __shared__ __align__(16) uint32_t s_w[4][kSlotDwords];
  __shared__ int s_sid[R];
  __shared__ float s_tw[R];  // with mul: the row's top-k weight rounded to bf16
  __shared__ int s_e[kPfScanSlab];
  __shared__ int s_tile;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int ntp = p.ntp[0];
  if (ntp > p.sorted_len) ntp = p.sorted_len;
  const int nblocks = ntp / p.bs;
  if (ty >= nblocks) return;  // a tile starts at a distinct block
  const int per_tile = R / p.bs;  // m-blocks per R-row tile (>= 1)

  int mb = -1;
  if (nblocks <= kPfScanSlab) {
    for (int i = tid; i < nblocks; i += blockDim.x) s_e[i] = p.expert_ids[i];
    if (tid == 0) s_tile = -1;
    __syncthreads();
    if (wave == 0) {
      // pass 0 counts the tiles with all their blocks, pass 1 the others; an
      // expert's blocks are contiguous, so a tile is whole when its last block
      // has the leader's expert
      int k = ty;
      for (int pass = 0; pass < 2 && k >= 0; ++pass) {
        int run_start = 0, prev_e = -1;
        for (int w0 = 0; w0 < nblocks; w0 += 64) {
          const int blk = w0 + lane;
          const bool in = blk < nblocks;
          const int e = in ? s_e[blk] : -1;
          const int ep = lane > 0 ? s_e[blk - 1] : prev_e;
          const uint64_t starts = __ballot(in && (blk == 0 || e != ep));
          const uint64_t upto = starts & ((2ull << lane) - 1ull);
          const int run = upto ? w0 + 63 - __builtin_clzll(upto) : run_start;
          const bool lead = in && e >= 0 && e < p.num_experts && (blk - run) % per_tile == 0;
          const int last = blk + per_tile - 1;
          const bool whole = last < nblocks && s_e[last] == e;
          uint64_t leads = __ballot(lead && whole == (pass == 0));
          const int cnt = __builtin_popcountll(leads);
          if (k < cnt) {
            for (int q = k; q > 0; --q) leads &= leads - 1ull;
            if (lane == 0) s_tile = w0 + __builtin_ctzll(leads);
            k = -1;
            break;
          }
          k -= cnt;
          if (starts) run_start = w0 + 63 - __builtin_clzll(starts);
          prev_e = s_e[min(w0 + 63, nblocks - 1)];
        }
      }
    }
    __syncthreads();
    mb = s_tile;
  }
  // Wave 0 carries the scan state across 64-block windows and slabs.
  int tiles_before = 0;   // tiles starting before the current window
  int run_start = 0;      // first block of the run the window starts in
  int prev_e = -1;        // expert of the block before the window (none at block 0)
  if (nblocks > kPfScanSlab)
  for (int b0 = 0; b0 < nblocks; b0 += kPfScanSlab) {
    const int n = min(kPfScanSlab, nblocks - b0);
    __syncthreads();  // the previous slab is no longer read
    for (int i = tid; i < n; i += blockDim.x) s_e[i] = p.expert_ids[b0 + i];
    if (tid == 0) s_tile = -1;
    __syncthreads();
    if (wave == 0) {
      for (int w0 = 0; w0 < n; w0 += 64) {
        const int i = w0 + lane;
        const int blk = b0 + i;
        const bool in = i < n;
        const int e = in ? s_e[i] : -1;
        const int ep = i > w0 ? s_e[i - 1] : prev_e;
        const uint64_t starts = __ballot(in && (blk == 0 || e != ep));
        const uint64_t upto = starts & ((2ull << lane) - 1ull);
        const int run = upto ? b0 + w0 + 63 - __builtin_clzll(upto) : run_start;
        const bool lead = in && e >= 0 && e < p.num_experts && (blk - run) % per_tile == 0;
        uint64_t leads = __ballot(lead);
        const int cnt = __builtin_popcountll(leads);
        if (ty - tiles_before < cnt) {
          for (int k = ty - tiles_before; k > 0; --k) leads &= leads - 1ull;
          if (lane == 0) s_tile = b0 + w0 + __builtin_ctzll(leads);
          break;
        }
        tiles_before += cnt;
        if (starts) run_start = b0 + w0 + 63 - __builtin_clzll(starts);
        prev_e = s_e[min(w0 + 63, n - 1)];
      }
    }
    __syncthreads();
    mb = s_tile;
    if (mb >= 0) break;
  }
  if (mb < 0) return;  // past the last tile
  const int expert = __builtin_amdgcn_readfirstlane(p.expert_ids[mb]);
  // blocks of this tile: up to per_tile, while the expert stays the same
  const bool same = lane > 0 && lane < per_tile && mb + lane < nblocks &&
                    p.expert_ids[mb + lane] == expert;
  const uint64_t differ = ~__ballot(same) & ~1ull;  // bit 0: the leader itself
  const int nb = min(per_tile, static_cast<int>(__builtin_ctzll(differ)));
  const int rows = nb * p.bs;

  const int valid_limit = p.size_m * p.top_k;
  for (int r = tid; r < R; r += blockDim.x) {
    const int sid = (r < rows) ? p.sorted_ids[mb * p.bs + r] : valid_limit;
    s_sid[r] = sid;
    s_tw[r] = (p.mul && static_cast<unsigned>(sid) < static_cast<unsigned>(valid_limit))
                  ? bf2f(f2bf(p.topk_w[sid]))
                  : 0.0f;
  }
  __syncthreads();

  // 32-row blocks past the last routed row of the tile are skipped (an
  // expert's padding sits at the end of its segment, so for the routing
  // kernels' output this drops exactly the padding blocks).
  const uint64_t lo_rows = __ballot(s_sid[lane] < valid_limit);
  const uint64_t hi_rows = R > 64 ? __ballot(s_sid[(64 + lane) % R] < valid_limit) : 0ull;
  const int row_end = hi_rows ? 128 - __builtin_clzll(hi_rows)
                              : (lo_rows ? 64 - __builtin_clzll(lo_rows) : 0);
  // Column tiles of the four waves: four consecutive tiles, or with SwiGLU two
  // gate tiles (waves 0, 1) and their up tiles (waves 2, 3).
  int nt;
  bool tile_ok;
  if (p.act != nullptr) {
    const int gate = tx * 2 + (wave & 1);
    tile_ok = gate < (p.inter >> 6);
    nt = wave < 2 ? gate : gate + (p.inter >> 6);
  } else {
    nt = tx * 4 + wave;
    tile_ok = nt < (p.size_n >> 6);
  }
  const int rb = tile_ok ? __builtin_amdgcn_readfirstlane((row_end + 31) >> 5) : 0;
  uint32_t* s_w_wave = s_w[wave];
  if constexpr (R == 64) {
    switch (rb) {
      case 0: prefill_tile<0, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      case 1: prefill_tile<1, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      default: prefill_tile<2, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
    }
  } else {
    switch (rb) {
      case 0: prefill_tile<0, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      case 1: prefill_tile<1, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      case 2: prefill_tile<2, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      case 3: prefill_tile<3, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
      default: prefill_tile<4, R>(p, s_a, s_w_wave, s_sid, s_tw, expert, nt, tx); break;
    }
  }
}

template <int R>
__global__ __launch_bounds__(256, 2) void wna16_prefill_kernel(GemmArgs p) {
  prefill_block<R>(p, blockIdx.x, blockIdx.y);
}

// Two independent problems in one launch (e.g. a layer's routed experts and
// its shared expert): the flat grid holds the first problem's x0-by-y
// workgroups, then the second's, each in its own x-fastest order, so one
// stream keeps both on the GPU at once.
template <int R>
__global__ __launch_bounds__(256, 2) void wna16_prefill_pair_kernel(
    GemmArgs p0, GemmArgs p1, int x0, int n0, int x1) {
  const int l = static_cast<int>(blockIdx.x);
  if (l < n0)
    prefill_block<R>(p0, l % x0, l / x0);
  else
    prefill_block<R>(p1, (l - n0) % x1, (l - n0) / x1);
}

// W13 finish fused with SwiGLU: for every routed row, the gate and up
// columns are the sums of the K shares' fp32 partials (share order, so the
// result does not depend on scheduling), rounded to bf16 exactly as the W13
// output would be, then SwiGLU as in kimi_marlin_w13_swiglu_cuda.  One thread
// per 2 columns of a row, and all S >= splits shares' loads are issued before
// the first add (shares past the last re-read it and are not added), so the
// kernel costs one memory round trip whatever the share count.
template <int S>
__global__ void w13_swiglu_partials_kernel(GemmArgs p, uint16_t* __restrict__ act, int inter) {
  int ntp = p.ntp[0];
  if (ntp > p.sorted_len) ntp = p.sorted_len;
  const int per_row = inter >> 1;
  const int N = p.size_n;
  const int valid_limit = p.size_m * p.top_k;
  const long long total = static_cast<long long>(ntp) * per_row;
  const long long share = static_cast<long long>(valid_limit) * N;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const int pos = static_cast<int>(idx / per_row);
    const int c2 = static_cast<int>(idx - static_cast<long long>(pos) * per_row) * 2;
    // the row's id and its block's expert go out together
    const int sid = p.sorted_ids[pos];
    const int e = p.expert_ids[pos / p.bs];
    if (static_cast<unsigned>(sid) >= static_cast<unsigned>(valid_limit)) continue;
    if (e < 0 || e >= p.num_experts) continue;
    const float* base = p.partial + static_cast<long long>(sid) * N + c2;
    float2 gv[S], uv[S];
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      const long long off = static_cast<long long>(min(sp, p.splits - 1)) * share;
      gv[sp] = *reinterpret_cast<const float2*>(base + off);
      uv[sp] = *reinterpret_cast<const float2*>(base + off + inter);
    }
    float g0 = 0.0f, g1 = 0.0f, u0 = 0.0f, u1 = 0.0f;
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      // a select, not a branch: the loads above stay ahead of every add
      const bool use = sp < p.splits;
      g0 = use ? g0 + gv[sp].x : g0;
      g1 = use ? g1 + gv[sp].y : g1;
      u0 = use ? u0 + uv[sp].x : u0;
      u1 = use ? u1 + uv[sp].y : u1;
    }
    const uint32_t lo = swiglu_one(bf2f(f2bf(g0)), bf2f(f2bf(u0)));
    const uint32_t hi = swiglu_one(bf2f(f2bf(g1)), bf2f(f2bf(u1)));
    *reinterpret_cast<uint32_t*>(act + static_cast<long long>(sid) * inter + c2) = lo | (hi << 16);
  }
}

bool valid_block_size(int bs) { return bs == 8 || (bs >= 16 && bs <= 64 && bs % 16 == 0); }

// Prefill tile height: 64 rows when the routes could fill at most 64 rows per
// expert on average, else 128.  Few rows per expert leave the 128-row tiles
// mostly one or two 32-row blocks anyway, while a problem's large experts (a
// shared expert in the same pair launch) would get tiles twice as long as the
// rest, which then set the launch's last round.
bool small_prefill_tiles(long long routes, long long experts) { return routes <= 64LL * experts; }

// The kernels address one expert's weights and the activations through
// 32-bit buffer ranges.  The activation range must also stay at or below
// 2^31 bytes: offset 0x80000000 is how rows not routed here read zeros.
bool ranges_fit(long long size_m, long long size_n, long long size_k) {
  return size_n * size_k / 2 <= 0xffffffffLL && size_m * size_k * 2 <= 0x80000000LL;
}

}  // namespace

int wna16_gemm(const uint16_t* input, uint16_t* output, float* c_tmp, long long c_tmp_len,
               const uint8_t* b_qweight, const uint16_t* b_scales, int32_t* workspace,
               int workspace_len, const int32_t* sorted_token_ids, const int32_t* expert_ids,
               const int32_t* num_tokens_post_padded, const float* topk_weights,
               int sorted_token_ids_len, int moe_block_size, int top_k, bool mul_topk_weights,
               int size_m, int size_n, int size_k, int local_experts, int group_size,
               int cu_count, hipStream_t stream) {
  if (!input || !output || !b_qweight || !b_scales || !sorted_token_ids || !expert_ids ||
      !num_tokens_post_padded || !topk_weights)
    return fail(kInvalidValue, "wna16_gemm: null pointer");
  if (group_size != 32 || top_k <= 0 || size_m <= 0 || size_n <= 0 || size_k <= 0 ||
      sorted_token_ids_len <= 0 || local_experts <= 0)
    return fail(kInvalidValue, "wna16_gemm: bad shape m=%d n=%d k=%d topk=%d group=%d", size_m,
                size_n, size_k, top_k, group_size);
  if (!valid_block_size(moe_block_size))
    return fail(kInvalidValue, "wna16_gemm: moe_block_size %d not in {8,16,32,48,64}",
                moe_block_size);
  if (size_k % 32 != 0 || size_n % 64 != 0)
    return fail(kInvalidValue, "wna16_gemm: size_k %% 32 and size_n %% 64 must be 0 (k=%d n=%d)",
                size_k, size_n);
  if (moe_block_size > 16 && size_k % 64 != 0)
    return fail(kNotSupported, "wna16_gemm: the prefill tile kernel needs size_k %% 64 == 0 "
                "(k=%d)", size_k);
  if ((reinterpret_cast<uintptr_t>(input) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(output) & 15u) != 0)
    return fail(kInvalidValue, "wna16_gemm: input and output must be 16-byte aligned");
  if (static_cast<long long>(size_m) * top_k > 0x7fffffffLL)
    return fail(kInvalidValue, "wna16_gemm: size_m * top_k overflows int32");
  if (!ranges_fit(size_m, size_n, size_k))
    return fail(kNotSupported, "wna16_gemm: one expert's weights over 4 GiB or the input over "
                "2 GiB (m=%d n=%d k=%d)", size_m, size_n, size_k);
  if (cu_count <= 0) cu_count = current_cu_count();
  if (cu_count <= 0) return fail(kInvalidValue, "wna16_gemm: no device");

  const int max_m_blocks = ceil_div(sorted_token_ids_len, moe_block_size);
  const int n_tiles = size_n / 64;
  GemmArgs args{input, output, c_tmp, reinterpret_cast<const uint32_t*>(b_qweight), b_scales,
                workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
                sorted_token_ids_len, moe_block_size, top_k, mul_topk_weights ? 1 : 0, size_m,
                size_n, size_k, local_experts, 1, nullptr};

  if (moe_block_size <= 16) {
    // Decode: one workgroup per (m-block, tile).  Fewer expected workgroups ->
    // more waves per workgroup splitting K, so the chip stays busy.
    const int groups = size_k / 32;
    const long long routes = static_cast<long long>(size_m) * top_k;
    const long long est_blocks = routes < max_m_blocks ? routes : max_m_blocks;
    const long long wgs = est_blocks * n_tiles;
    int wk = wgs >= 4LL * cu_count ? 4 : (wgs >= 2LL * cu_count ? 8 : 16);
    while (wk > 4 && groups < wk) wk >>= 1;  // waves past the last group idle
    if (max_m_blocks > 65535) return fail(kNotSupported, "wna16_gemm: too many m-blocks");
    if (wk == 4) launch_decode<4>(args, max_m_blocks, stream);
    else if (wk == 8) launch_decode<8>(args, max_m_blocks, stream);
    else launch_decode<16>(args, max_m_blocks, stream);
    return launch_status("wna16_gemm (decode)");
  }
  if (max_m_blocks > 65535) return fail(kNotSupported, "wna16_gemm: too many m-blocks");
  const dim3 grid(ceil_div(n_tiles, 4), max_m_blocks);
  if (small_prefill_tiles(static_cast<long long>(size_m) * top_k, local_experts))
    hipLaunchKernelGGL(wna16_prefill_kernel<64>, grid, dim3(256), 0, stream, args);
  else
    hipLaunchKernelGGL(wna16_prefill_kernel<128>, grid, dim3(256), 0, stream, args);
  return launch_status("wna16_gemm (prefill)");
}

// W13 GEMM + SwiGLU for the small-batch decode path (block size <= 16).  The
// few (m-block, tile) workgroups of a small batch are multiplied by splitting
// K across workgroups; their fp32 partials go to `partials` and the SwiGLU
// kernel sums them, so the split costs no extra launch and no cross-workgroup
// synchronisation.  The share count is capped by what `partials` holds, and a
// buffer that cannot hold two shares runs the launch unsplit; the bits then
// depend only on `partials_len`, whichever entry point supplies the buffer.
int wna16_w13_swiglu(const uint16_t* input, uint16_t* act, float* partials, long long partials_len,
                     const uint8_t* b_qweight, const uint16_t* b_scales,
                     const int32_t* sorted_token_ids, const int32_t* expert_ids,
                     const int32_t* num_tokens_post_padded, int sorted_token_ids_len,
                     int moe_block_size, int top_k, int size_m, int inter, int size_k,
                     int local_experts, int group_size, int cu_count, hipStream_t stream) {
  if (!input || !act || !b_qweight || !b_scales || !sorted_token_ids || !expert_ids ||
      !num_tokens_post_padded)
    return fail(kInvalidValue, "w13_swiglu: null pointer");
  if (group_size != 32 || top_k <= 0 || size_m <= 0 || inter <= 0 || size_k <= 0 ||
      sorted_token_ids_len <= 0 || local_experts <= 0)
    return fail(kInvalidValue, "w13_swiglu: bad shape m=%d inter=%d k=%d", size_m, inter, size_k);
  if (!valid_block_size(moe_block_size))
    return fail(kInvalidValue, "w13_swiglu: block size %d not in {8, 16, 32, 48, 64}",
                moe_block_size);
  const int size_n = 2 * inter;
  if (size_k % 32 != 0 || inter % 64 != 0)
    return fail(kInvalidValue, "w13_swiglu: size_k %% 32 and inter %% 64 must be 0");
  if (moe_block_size > 16 && size_k % 64 != 0)
    return fail(kNotSupported, "w13_swiglu: the prefill tile kernel needs size_k %% 64 == 0");
  if ((reinterpret_cast<uintptr_t>(input) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(act) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(partials) & 15u) != 0)
    return fail(kInvalidValue, "w13_swiglu: input, act and partials must be 16-byte aligned");
  if (static_cast<long long>(size_m) * top_k > 0x7fffffffLL)
    return fail(kInvalidValue, "w13_swiglu: size_m * top_k overflows int32");
  if (!ranges_fit(size_m, size_n, size_k))
    return fail(kNotSupported, "w13_swiglu: one expert's weights over 4 GiB or the input over "
                "2 GiB (m=%d inter=%d k=%d)", size_m, inter, size_k);
  const int max_m_blocks = ceil_div(sorted_token_ids_len, moe_block_size);
  if (max_m_blocks > 65535) return fail(kNotSupported, "w13_swiglu: too many m-blocks");
  if (moe_block_size > 16) {
    // Prefill: the tile GEMM with the SwiGLU epilogue (partials not used).
    GemmArgs args{input, nullptr, nullptr, reinterpret_cast<const uint32_t*>(b_qweight),
                  b_scales, nullptr, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  nullptr, sorted_token_ids_len, moe_block_size, top_k, 0, size_m, size_n,
                  size_k, local_experts, 1, nullptr, act, inter};
    const dim3 grid(ceil_div(inter / 64, 2), max_m_blocks);
    if (small_prefill_tiles(static_cast<long long>(size_m) * top_k, local_experts))
      hipLaunchKernelGGL(wna16_prefill_kernel<64>, grid, dim3(256), 0, stream, args);
    else
      hipLaunchKernelGGL(wna16_prefill_kernel<128>, grid, dim3(256), 0, stream, args);
    return launch_status("w13_swiglu (prefill)");
  }
  if (cu_count <= 0) cu_count = current_cu_count();
  if (cu_count <= 0) return fail(kInvalidValue, "w13_swiglu: no device");
  const long long routes = static_cast<long long>(size_m) * top_k;
  const int n_tiles = size_n / 64;
  const int groups = size_k / 32;
  const long long est_blocks = routes < max_m_blocks ? routes : max_m_blocks;
  const long long wgs = est_blocks * n_tiles;
  // shares: about two workgroups per CU, at least 8 groups (two per wave) each,
  // as many as the partials buffer holds
  long long sp = (2LL * cu_count + wgs - 1) / wgs;
  if (sp > 16) sp = 16;
  if (sp > groups / 8) sp = groups / 8;
  const long long cap = partials ? partials_len / (routes * size_n) : 0;
  if (sp > cap) sp = cap;
  if (sp <= 1) {
    // No K split: a gate tile and its up tile in one workgroup of 2 WK waves,
    // SwiGLU in the epilogue (partials not used).
    GemmArgs args{input, nullptr, nullptr, reinterpret_cast<const uint32_t*>(b_qweight),
                  b_scales, nullptr, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  nullptr, sorted_token_ids_len, moe_block_size, top_k, 0, size_m, size_n,
                  size_k, local_experts, 1, nullptr, act, inter};
    const long long pair_wgs = est_blocks * (inter / 64);
    int wk = pair_wgs >= 2LL * cu_count ? 4 : 8;
    while (wk > 4 && groups < 2 * wk) wk >>= 1;  // keep >= 2 groups per wave
    if (wk == 4) launch_decode_pair<4>(args, max_m_blocks, stream);
    else launch_decode_pair<8>(args, max_m_blocks, stream);
    return launch_status("w13_swiglu (decode)");
  }
  const int splits = static_cast<int>(sp);
  GemmArgs args{input, nullptr, nullptr, reinterpret_cast<const uint32_t*>(b_qweight), b_scales,
                nullptr, sorted_token_ids, expert_ids, num_tokens_post_padded, nullptr,
                sorted_token_ids_len, moe_block_size, top_k, 0, size_m, size_n, size_k,
                local_experts, splits, partials};
  const long long total_wgs = wgs * splits;
  int wk = total_wgs >= 4LL * cu_count ? 4 : (total_wgs >= 2LL * cu_count ? 8 : 16);
  while (wk > 4 && groups / splits < 2 * wk) wk >>= 1;  // keep >= 2 groups per wave
  if (wk == 4) launch_decode<4>(args, max_m_blocks, stream);
  else if (wk == 8) launch_decode<8>(args, max_m_blocks, stream);
  else launch_decode<16>(args, max_m_blocks, stream);
  const int rc = launch_status("w13_swiglu (GEMM)");
  if (rc != kSuccess) return rc;
  const long long work = static_cast<long long>(sorted_token_ids_len) * (inter / 2);
  long long grid = (work + 255) / 256;
  if (grid > 4LL * cu_count) grid = 4LL * cu_count;
  const dim3 g(static_cast<unsigned>(grid));
  if (splits <= 4)
    hipLaunchKernelGGL(w13_swiglu_partials_kernel<4>, g, dim3(256), 0, stream, args, act, inter);
  else if (splits <= 8)
    hipLaunchKernelGGL(w13_swiglu_partials_kernel<8>, g, dim3(256), 0, stream, args, act, inter);
  else
    hipLaunchKernelGGL(w13_swiglu_partials_kernel<16>, g, dim3(256), 0, stream, args, act, inter);
  return launch_status("w13_swiglu (SwiGLU)");
}

namespace {

// Checks one problem of the pair entry and fills its kernel arguments and its
// (column groups, m-blocks) grid.
int prefill_problem(const pega_wna16_problem* q, const char* which, GemmArgs& args, int& gx,
                    int& gy) {
  if (!q) return fail(kInvalidValue, "wna16_prefill_pair: %s problem is NULL", which);
  const bool swiglu = q->act != nullptr;
  if (!q->input || (!swiglu && !q->output) || !q->b_qweight || !q->b_scales ||
      !q->sorted_token_ids || !q->expert_ids || !q->num_tokens_post_padded ||
      (q->mul_topk_weights && !q->topk_weights))
    return fail(kInvalidValue, "wna16_prefill_pair: %s problem has a null pointer", which);
  if (q->group_size != 32 || q->top_k <= 0 || q->size_m <= 0 || q->size_n <= 0 ||
      q->size_k <= 0 || q->sorted_token_ids_len <= 0 || q->local_experts <= 0 ||
      (q->mul_topk_weights != 0 && q->mul_topk_weights != 1))
    return fail(kInvalidValue, "wna16_prefill_pair: %s problem has a bad shape m=%d n=%d k=%d",
                which, q->size_m, q->size_n, q->size_k);
  if (q->moe_block_size != 32 && q->moe_block_size != 48 && q->moe_block_size != 64)
    return fail(kNotSupported, "wna16_prefill_pair: %s problem's block size %d is not 32, 48 "
                "or 64", which, q->moe_block_size);
  if (q->size_k % 64 != 0 || q->size_n % (swiglu ? 128 : 64) != 0)
    return fail(kNotSupported, "wna16_prefill_pair: %s problem needs size_k %% 64 and size_n %% "
                "%d == 0 (k=%d n=%d)", which, swiglu ? 128 : 64, q->size_k, q->size_n);
  if (swiglu && q->mul_topk_weights)
    return fail(kInvalidValue, "wna16_prefill_pair: %s problem: the SwiGLU epilogue applies no "
                "top-k weight", which);
  const void* out = swiglu ? static_cast<const void*>(q->act) : q->output;
  if ((reinterpret_cast<uintptr_t>(q->input) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(out) & 15u) != 0)
    return fail(kInvalidValue, "wna16_prefill_pair: %s problem's input and output must be "
                "16-byte aligned", which);
  if (static_cast<long long>(q->size_m) * q->top_k > 0x7fffffffLL)
    return fail(kInvalidValue, "wna16_prefill_pair: %s problem: size_m * top_k overflows int32",
                which);
  if (!ranges_fit(q->size_m, q->size_n, q->size_k))
    return fail(kNotSupported, "wna16_prefill_pair: %s problem: one expert's weights over 4 GiB "
                "or the input over 2 GiB", which);
  const int inter = q->size_n / 2;
  args = GemmArgs{q->input, swiglu ? nullptr : q->output, nullptr,
                  reinterpret_cast<const uint32_t*>(q->b_qweight), q->b_scales, nullptr,
                  q->sorted_token_ids, q->expert_ids, q->num_tokens_post_padded,
                  q->topk_weights, q->sorted_token_ids_len, q->moe_block_size, q->top_k,
                  q->mul_topk_weights, q->size_m, q->size_n, q->size_k, q->local_experts, 1,
                  nullptr, swiglu ? q->act : nullptr, swiglu ? inter : 0};
  gx = swiglu ? ceil_div(inter / 64, 2) : ceil_div(q->size_n / 64, 4);
  gy = ceil_div(q->sorted_token_ids_len, q->moe_block_size);
  return kSuccess;
}

}  // namespace

int wna16_prefill_pair(const pega_wna16_problem* first, const pega_wna16_problem* second,
                       hipStream_t stream) {
  GemmArgs a0, a1;
  int x0, y0, x1, y1;
  int rc = prefill_problem(first, "first", a0, x0, y0);
  if (rc != kSuccess) return rc;
  rc = prefill_problem(second, "second", a1, x1, y1);
  if (rc != kSuccess) return rc;
  const long long n0 = static_cast<long long>(x0) * y0, n1 = static_cast<long long>(x1) * y1;
  if (n0 + n1 > 0x7fffffffLL)
    return fail(kNotSupported, "wna16_prefill_pair: %lld workgroups exceed the grid", n0 + n1);
  // one tile height for both problems, from their routes and experts together
  const long long routes = static_cast<long long>(a0.size_m) * a0.top_k +
                           static_cast<long long>(a1.size_m) * a1.top_k;
  const dim3 grid(static_cast<unsigned>(n0 + n1));
  if (small_prefill_tiles(routes, static_cast<long long>(a0.num_experts) + a1.num_experts))
    hipLaunchKernelGGL(wna16_prefill_pair_kernel<64>, grid, dim3(256), 0, stream, a0, a1, x0,
                       static_cast<int>(n0), x1);
  else
    hipLaunchKernelGGL(wna16_prefill_pair_kernel<128>, grid, dim3(256), 0, stream, a0, a1, x0,
                       static_cast<int>(n0), x1);
  return launch_status("wna16_prefill_pair");
}

}  // namespace pega

// ---------------------------------------------------------------- C ABI
// Reference: pegainfer-kernels/src/ffi/kimi.rs:131-152; launcher guards
// csrc/kimi_k2/kimi_marlin_wna16.cu:264-309 (local_experts == 48,
// group_size == 32, block size set, c_tmp and workspace required).  The split
// K reduction happens inside each workgroup, so c_tmp and the lock workspace
// are validated but never read or written (a caller's zero-filled locks stay
// zero).
PEGA_API int kimi_marlin_wna16_gemm_cuda(
    const uint16_t* input, uint16_t* output, float* c_tmp, const uint8_t* b_qweight,
    const uint16_t* b_scales, int32_t* workspace, const int32_t* sorted_token_ids,
    const int32_t* expert_ids, const int32_t* num_tokens_post_padded, const float* topk_weights,
    int workspace_len, int sorted_token_ids_len, int moe_block_size, int top_k,
    bool mul_topk_weights, int size_m, int size_n, int size_k, int local_experts, int group_size,
    int sm_count, hipStream_t stream) {
  // the reference's checks, in its order (kimi_marlin_wna16.cu:264-309)
  if (!input || !output || !b_qweight || !b_scales || !workspace || !sorted_token_ids ||
      !expert_ids || !num_tokens_post_padded || !topk_weights)
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: null pointer");
  if (!c_tmp) return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: c_tmp is required");
  if (local_experts != 48 || group_size != 32 || top_k <= 0 || size_m <= 0 || size_n <= 0 ||
      size_k <= 0 || sorted_token_ids_len <= 0)
    return pega::fail(pega::kInvalidValue,
                      "kimi wna16_gemm: bad shape (experts=%d group=%d topk=%d m=%d n=%d k=%d)",
                      local_experts, group_size, top_k, size_m, size_n, size_k);
  if (!pega::valid_block_size(moe_block_size))
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: moe_block_size %d not in "
                      "{8,16,32,48,64}", moe_block_size);
  if (size_k % 16 != 0 || size_n % 64 != 0 || size_k % group_size != 0)
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: bad k/n (k=%d n=%d)", size_k,
                      size_n);
  // the lock-workspace floor (:305-309), sm_count <= 0 meaning the device's CU count; the
  // locks are not used here, but a caller that sized them too small is rejected the same way
  int cus = sm_count;
  if (cus <= 0) cus = pega::current_cu_count();
  if (cus <= 0) return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: no device");
  const long long min_ws = std::min(static_cast<long long>(size_n / 64) *
                                        (sorted_token_ids_len / moe_block_size),
                                    4LL * cus);
  if (workspace_len < min_ws)
    return pega::fail(pega::kInvalidValue,
                      "kimi wna16_gemm: workspace_len %d below min(n_tiles * m_blocks, 4 * "
                      "sm_count) = %lld", workspace_len, min_ws);
  const long long c_tmp_len = static_cast<long long>(size_n) * sorted_token_ids_len *
                              (moe_block_size == 8 ? 2 : 1);
  return pega::wna16_gemm(input, output, c_tmp, c_tmp_len, b_qweight, b_scales, workspace,
                          workspace_len, sorted_token_ids, expert_ids, num_tokens_post_padded,
                          topk_weights, sorted_token_ids_len, moe_block_size, top_k,
                          mul_topk_weights, size_m, size_n, size_k, local_experts, group_size,
                          sm_count, stream);
}

// Shape-general entry (any expert count; expert ids outside [0, local_experts)
// are skipped; c_tmp / workspace may be null).  No reference counterpart: the
// reference accepts 48 experts only.
PEGA_API int pega_wna16_gemm(const uint16_t* input, uint16_t* output, float* c_tmp,
                             long long c_tmp_len, const uint8_t* b_qweight,
                             const uint16_t* b_scales, int32_t* workspace, int workspace_len,
                             const int32_t* sorted_token_ids, const int32_t* expert_ids,
                             const int32_t* num_tokens_post_padded, const float* topk_weights,
                             int sorted_token_ids_len, int moe_block_size, int top_k,
                             bool mul_topk_weights, int size_m, int size_n, int size_k,
                             int local_experts, int group_size, int sm_count,
                             hipStream_t stream) {
  return pega::wna16_gemm(input, output, c_tmp, c_tmp_len, b_qweight, b_scales, workspace,
                          workspace_len, sorted_token_ids, expert_ids, num_tokens_post_padded,
                          topk_weights, sorted_token_ids_len, moe_block_size, top_k,
                          mul_topk_weights, size_m, size_n, size_k, local_experts, group_size,
                          sm_count, stream);
}

// Fused W13 + SwiGLU for the small-batch decode path (no reference symbol: the
// reference runs kimi_marlin_wna16_gemm_cuda then kimi_marlin_w13_swiglu_cuda).
PEGA_API int pega_wna16_w13_swiglu(const uint16_t* input, uint16_t* act, float* partials,
                                   long long partials_len, const uint8_t* b_qweight,
                                   const uint16_t* b_scales, const int32_t* sorted_token_ids,
                                   const int32_t* expert_ids,
                                   const int32_t* num_tokens_post_padded,
                                   int sorted_token_ids_len, int moe_block_size, int top_k,
                                   int size_m, int intermediate_dim, int size_k, int local_experts,
                                   int group_size, int sm_count, hipStream_t stream) {
  return pega::wna16_w13_swiglu(input, act, partials, partials_len, b_qweight, b_scales,
                                sorted_token_ids, expert_ids, num_tokens_post_padded,
                                sorted_token_ids_len, moe_block_size, top_k, size_m,
                                intermediate_dim, size_k, local_experts, group_size, sm_count,
                                stream);
}

// ---------------------------------------------------------------- no-allocation variant
// The K-split partials of pega_wna16_w13_swiglu live in this fixed device array
// instead of a caller workspace: 2 MiB (524,288 floats) per device, held until the
// process ends.  Host code never passes `scratch` itself to a kernel (in host code the
// name is only a stand-in for the device symbol): its device address is looked up once
// per device, with that device current, and kept in g_scratch_addr.
namespace {
constexpr long long kScratchFloats = 1LL << 19;
std::atomic<float*> g_scratch_addr[64];
}  // namespace
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
// This device's address of `scratch` (looked up on the first call on the device).
// The kernels run on `stream`'s device, so that device must be the current one
// (the lookup returns the current device's copy of the array).
float* scratch_address(hipStream_t stream, int* status) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *status = pega::fail(pega::kInvalidValue, "w13_swiglu (no-alloc): no current device");
    return nullptr;
  }
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) {
      *status = pega::fail(pega::kInvalidValue, "w13_swiglu (no-alloc): the stream belongs to "
                           "device %d, not to the current device %d", sdev, dev);
      return nullptr;
    }
  }
  float* ptr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (ptr != nullptr) return ptr;
  void* addr = nullptr;
  const hipError_t err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (err != hipSuccess || addr == nullptr) {
    *status = pega::fail(pega::kLaunchFailed, "w13_swiglu (no-alloc): hipGetSymbolAddress: %s",
                         hipGetErrorString(err));
    return nullptr;
  }
  ptr = static_cast<float*>(addr);
  g_scratch_addr[dev].store(ptr, std::memory_order_release);
  return ptr;
}
}  // namespace

// pega_wna16_w13_swiglu without the partials workspace (no reference counterpart; for
// callers that cannot allocate, e.g. code under HIP graph capture): the K-split partials
// go to the library's static per-device scratch.  Nothing in it needs clearing: every
// routed row of every share is written before the SwiGLU kernel reads it.  Calls that
// overlap on one device race on the scratch.  The output equals pega_wna16_w13_swiglu's
// with a partials workspace of the scratch's size (524,288 floats): as there, a split the
// scratch cannot hold two shares of runs unsplit.  The current device must own `stream`.
PEGA_API int pega_wna16_w13_swiglu_noalloc(const uint16_t* input, uint16_t* act,
                                           const uint8_t* b_qweight, const uint16_t* b_scales,
                                           const int32_t* sorted_token_ids,
                                           const int32_t* expert_ids,
                                           const int32_t* num_tokens_post_padded,
                                           int sorted_token_ids_len, int moe_block_size,
                                           int top_k, int size_m, int intermediate_dim,
                                           int size_k, int local_experts, int group_size,
                                           int sm_count, hipStream_t stream) {
  int status = pega::kSuccess;
  float* partials = scratch_address(stream, &status);
  if (partials == nullptr) return status;
  return pega::wna16_w13_swiglu(input, act, partials, kScratchFloats, b_qweight, b_scales,
                                sorted_token_ids, expert_ids, num_tokens_post_padded,
                                sorted_token_ids_len, moe_block_size, top_k, size_m,
                                intermediate_dim, size_k, local_experts, group_size, sm_count,
                                stream);
}

// Two prefill-size GEMMs in one launch (no reference symbol: the reference
// launches a layer's shared expert and its routed experts one after another).
PEGA_API int pega_wna16_prefill_pair(const pega_wna16_problem* first,
                                     const pega_wna16_problem* second, hipStream_t stream) {
  return pega::wna16_prefill_pair(first, second, stream);
}
