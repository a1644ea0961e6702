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
#include "common.h"

namespace pega {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16_t;

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
  return r;
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
                                                  const ColScale& b, uint32_t k1024,
                                                  uint32_t k64) {
  const uint32_t p0 = and_or(x, 0x000F000Fu, k1024);
  const uint32_t p1 = and_or(x, 0x00F000F0u, k64);
  const uint32_t y = x >> 8;
  const uint32_t p2 = and_or(y, 0x000F000Fu, k1024);
  const uint32_t p3 = and_or(y, 0x00F000F0u, k64);
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
                                         uint32_t k1024, uint32_t k64) {
  const ColScale a = col_scale(bf_lo(scale_pair));
  const ColScale b = col_scale(bf_hi(scale_pair));
  const WordPairs q0 = dequant_word(w[0], a, b, k1024, k64);
  const WordPairs q1 = dequant_word(w[1], a, b, k1024, k64);
  const WordPairs q2 = dequant_word(w[2], a, b, k1024, k64);
  const WordPairs q3 = dequant_word(w[3], a, b, k1024, k64);
  // slot order k = {0,1,2,3,8,9,10,11} (jj 0,1) and {4,...,15} (jj 2,3)
  BFrags f;
  f.x1 = as_bf16x8(q0.n0_lo, q1.n0_lo, q0.n0_hi, q1.n0_hi);
  f.x2 = as_bf16x8(q2.n0_lo, q3.n0_lo, q2.n0_hi, q3.n0_hi);
  f.y1 = as_bf16x8(q0.n1_lo, q1.n1_lo, q0.n1_hi, q1.n1_hi);
  f.y2 = as_bf16x8(q2.n1_lo, q3.n1_lo, q2.n1_hi, q3.n1_hi);
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
  int splits;       // cross-workgroup K splits (decode kernel)
};

__device__ __forceinline__ uint16_t epilogue_value(float acc, int sid, const GemmArgs& p) {
  uint16_t c = f2bf(acc);
  if (p.mul) c = f2bf(bf2f(c) * bf2f(f2bf(p.topk_w[sid])));
  return c;
}

// ---------------------------------------------------------------------------
// Decode kernel: one workgroup per (m-block, 64-column tile, K split), WK
// waves splitting the K range, rows <= 32 (one MFMA row block), activations
// read straight from global memory (only valid rows are loaded).
// ---------------------------------------------------------------------------
template <int WK>
__global__ __launch_bounds__(64 * WK) void wna16_decode_kernel(GemmArgs p) {
  __shared__ int s_sid[32];
  __shared__ float s_red[WK][32][64];
  __shared__ int s_last;

  const int n_tiles = p.size_n >> 6;
  const int nt = blockIdx.x % n_tiles;
  const int split = blockIdx.x / n_tiles;
  const int mb = blockIdx.y;
  int ntp = p.ntp[0];
  if (ntp > p.sorted_len) ntp = p.sorted_len;
  if (mb >= ntp / p.bs) return;  // whole blocks only: rows stay inside sorted_len
  const int expert = p.expert_ids[mb];
  if (expert < 0 || expert >= p.num_experts) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int valid_limit = p.size_m * p.top_k;
  if (tid < 32) {
    int sid = valid_limit;
    if (tid < p.bs) sid = p.sorted_ids[mb * p.bs + tid];
    s_sid[tid] = sid;
  }
  __syncthreads();

  const int c = lane & 31, h = lane >> 5;
  const int K = p.size_k, N = p.size_n;
  const int groups = K >> 5;
  const int slices = p.splits * WK;
  const int slice = split * WK + wave;
  const int g0 = (groups * slice) / slices, g1 = (groups * (slice + 1)) / slices;

  // activation row of this lane (row m = c)
  const int my_sid = s_sid[c];
  const bool row_ok = my_sid < valid_limit;
  const uint16_t* arow = p.input + static_cast<long long>(row_ok ? my_sid / p.top_k : 0) * K;

  const long long expert_words = static_cast<long long>(N) * (K >> 3);
  const uint32_t* wbase = p.qweight + expert * expert_words +
                          static_cast<long long>(nt) * 128 + 16 * (c & 7) + (c >> 3);
  const long long tile_row_words = static_cast<long long>(n_tiles) * 128;  // one k-tile row
  const uint32_t* sbase = reinterpret_cast<const uint32_t*>(
      p.scales + static_cast<long long>(expert) * (K >> 5) * N + nt * 64 + 8 * (c & 7) +
      2 * (c >> 3));
  const int srow_words = N >> 1;

  const uint32_t k1024 = 0x64006400u, k64 = 0x54005400u;
  floatx16_t accx = {}, accy = {};

  for (int g = g0; g < g1; ++g) {
    const uint32_t* wp = wbase + (2LL * g + h) * tile_row_words;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = wp[4 * j];
    const uint32_t sp = sbase[static_cast<long long>(g) * srow_words];
    uint4 a0 = make_uint4(0, 0, 0, 0), a1 = make_uint4(0, 0, 0, 0);
    if (row_ok) {
      const uint4* ap = reinterpret_cast<const uint4*>(arow + 32 * g + 16 * h);
      a0 = ap[0];
      a1 = ap[1];
    }
    const BFrags b = make_b(w, sp, k1024, k64);
    const bf16x8_t A1 = as_bf16x8(a0.x, a0.y, a1.x, a1.y);
    const bf16x8_t A2 = as_bf16x8(a0.z, a0.w, a1.z, a1.w);
    accx = mfma(A1, b.x1, accx);
    accx = mfma(A2, b.x2, accx);
    accy = mfma(A1, b.y1, accy);
    accy = mfma(A2, b.y2, accy);
  }

  // Deterministic reduction over the WK waves (fixed order 0..WK-1).
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s_red[wave][i][lane] = accx[i];
    s_red[wave][16 + i][lane] = accy[i];
  }
  __syncthreads();

  const int n0 = nt * 64 + (c >> 3) * 16 + (c & 7);
  // Each wave finalises 32/WK of the lane's 32 values.
  constexpr int kPer = 32 / WK;
  float v[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int j = wave * kPer + q;
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < WK; ++w) s += s_red[w][j][lane];
    v[q] = s;
  }

  if (p.splits > 1) {
    // Partial of this split -> c_tmp[split][mb*bs + row][n]; the last of the
    // splits to arrive sums the partials in split order and writes C.
    const long long rows_cap = p.sorted_len;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int j = wave * kPer + q;
      const int row = acc_row(j & 15, h);
      const int n = (j < 16) ? n0 : n0 + 8;
      if (row < p.bs)
        p.c_tmp[(split * rows_cap + mb * p.bs + row) * N + n] = v[q];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const int old = atomicAdd(&p.locks[mb * n_tiles + nt], 1);
      s_last = (old == p.splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int j = wave * kPer + q;
      const int row = acc_row(j & 15, h);
      const int n = (j < 16) ? n0 : n0 + 8;
      float s = 0.0f;
      if (row < p.bs)
        for (int sp = 0; sp < p.splits; ++sp)
          s += __builtin_nontemporal_load(&p.c_tmp[(sp * rows_cap + mb * p.bs + row) * N + n]);
      v[q] = s;
    }
    if (tid == 0) p.locks[mb * n_tiles + nt] = 0;
  }

#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int j = wave * kPer + q;
    const int row = acc_row(j & 15, h);
    const int n = (j < 16) ? n0 : n0 + 8;
    if (row < p.bs) {
      const int sid = s_sid[row];
      if (sid < valid_limit)
        p.output[static_cast<long long>(sid) * N + n] = epilogue_value(v[q], sid, p);
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill kernel: one workgroup per (leader m-block, 4 column tiles); the
// leader takes up to 128/bs consecutive m-blocks of the same expert (a
// 128-row tile), 4 waves each own one 64-column tile, the activation tile is
// staged in LDS per 64-wide K chunk (double buffered), weights go straight
// from global memory into registers and are dequantised there.
// ---------------------------------------------------------------------------
constexpr int kPfRows = 128;
constexpr int kPfChunk = 64;                 // k per LDS stage (2 quant groups)
constexpr int kPfLdsStride = kPfChunk + 8;   // bf16 per LDS row (padding vs bank conflicts)

__global__ __launch_bounds__(256, 2) void wna16_prefill_kernel(GemmArgs p) {
  __shared__ __align__(16) uint16_t s_a[2][kPfRows * kPfLdsStride];
  __shared__ int s_sid[kPfRows];
  __shared__ int s_seg_break;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mb = blockIdx.y;
  int ntp = p.ntp[0];
  if (ntp > p.sorted_len) ntp = p.sorted_len;
  const int nblocks = ntp / p.bs;
  if (mb >= nblocks) return;
  const int expert = p.expert_ids[mb];
  if (expert < 0 || expert >= p.num_experts) return;

  // Start of this expert's run of blocks: 1 + the last j < mb whose expert differs.
  if (tid == 0) s_seg_break = -1;
  __syncthreads();
  for (int j = tid; j < mb; j += blockDim.x)
    if (p.expert_ids[j] != expert) atomicMax(&s_seg_break, j);
  __syncthreads();
  const int seg_start = s_seg_break + 1;
  const int per_tile = kPfRows / p.bs;  // m-blocks per 128-row tile (>= 1)
  if ((mb - seg_start) % per_tile != 0) return;
  int nb = 1;
  while (nb < per_tile && mb + nb < nblocks && p.expert_ids[mb + nb] == expert) ++nb;
  const int rows = nb * p.bs;

  const int valid_limit = p.size_m * p.top_k;
  for (int r = tid; r < kPfRows; r += blockDim.x)
    s_sid[r] = (r < rows) ? p.sorted_ids[mb * p.bs + r] : valid_limit;
  __syncthreads();

  const int K = p.size_k, N = p.size_n;
  const int n_tiles = N >> 6;
  const int nt = blockIdx.x * 4 + wave;
  const bool wave_active = nt < n_tiles;
  const int c = lane & 31, h = lane >> 5;
  const long long expert_words = static_cast<long long>(N) * (K >> 3);
  const int ntc = wave_active ? nt : 0;
  const uint32_t* wbase = p.qweight + expert * expert_words + static_cast<long long>(ntc) * 128 +
                          16 * (c & 7) + (c >> 3);
  const long long tile_row_words = static_cast<long long>(n_tiles) * 128;
  const uint32_t* sbase = reinterpret_cast<const uint32_t*>(
      p.scales + static_cast<long long>(expert) * (K >> 5) * N + ntc * 64 + 8 * (c & 7) +
      2 * (c >> 3));
  const int srow_words = N >> 1;

  // Activation staging: 128 rows x 64 k = 1024 16-byte pieces, 4 per thread.
  uint4 stage[4];
  auto load_chunk = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = tid + 256 * i;
      const int r = piece >> 3, q = piece & 7;
      const int sid = s_sid[r];
      stage[i] = make_uint4(0, 0, 0, 0);
      if (sid < valid_limit)
        stage[i] = *reinterpret_cast<const uint4*>(
            p.input + static_cast<long long>(sid / p.top_k) * K + chunk * kPfChunk + 8 * q);
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = tid + 256 * i;
      const int r = piece >> 3, q = piece & 7;
      *reinterpret_cast<uint4*>(&s_a[buf][r * kPfLdsStride + 8 * q]) = stage[i];
    }
  };

  floatx16_t accx[4], accy[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    accx[rb] = floatx16_t{};
    accy[rb] = floatx16_t{};
  }
  const uint32_t k1024 = 0x64006400u, k64 = 0x54005400u;
  const int chunks = K / kPfChunk;

  load_chunk(0);
  store_chunk(0);
  __syncthreads();
  for (int ch = 0; ch < chunks; ++ch) {
    const int buf = ch & 1;
    if (ch + 1 < chunks) load_chunk(ch + 1);
    if (wave_active) {
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g = ch * 2 + gg;
        const uint32_t* wp = wbase + (2LL * g + h) * tile_row_words;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = wp[4 * j];
        const uint32_t sp = sbase[static_cast<long long>(g) * srow_words];
        const BFrags b = make_b(w, sp, k1024, k64);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const uint16_t* ap = &s_a[buf][(32 * rb + c) * kPfLdsStride + 32 * gg + 16 * h];
          const uint4 a0 = *reinterpret_cast<const uint4*>(ap);
          const uint4 a1 = *reinterpret_cast<const uint4*>(ap + 8);
          const bf16x8_t A1 = as_bf16x8(a0.x, a0.y, a1.x, a1.y);
          const bf16x8_t A2 = as_bf16x8(a0.z, a0.w, a1.z, a1.w);
          accx[rb] = mfma(A1, b.x1, accx[rb]);
          accx[rb] = mfma(A2, b.x2, accx[rb]);
          accy[rb] = mfma(A1, b.y1, accy[rb]);
          accy[rb] = mfma(A2, b.y2, accy[rb]);
        }
      }
    }
    if (ch + 1 < chunks) {
      // buf^1 was last read in iteration ch-1, which every wave finished
      // before the barrier that ended it; one barrier per chunk suffices.
      store_chunk(buf ^ 1);
      __syncthreads();
    }
  }

  if (!wave_active) return;
  const int n0 = nt * 64 + (c >> 3) * 16 + (c & 7);
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 32 * rb + acc_row(i, h);
      const int sid = s_sid[row];
      if (sid < valid_limit) {
        p.output[static_cast<long long>(sid) * N + n0] = epilogue_value(accx[rb][i], sid, p);
        p.output[static_cast<long long>(sid) * N + n0 + 8] = epilogue_value(accy[rb][i], sid, p);
      }
    }
  }
}

bool valid_block_size(int bs) { return bs == 8 || (bs >= 16 && bs <= 64 && bs % 16 == 0); }

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
  if (size_k % 64 != 0 || size_n % 64 != 0)
    return fail(kNotSupported, "wna16_gemm: size_k %% 64 and size_n %% 64 must be 0 (k=%d n=%d)",
                size_k, size_n);
  if ((reinterpret_cast<uintptr_t>(input) & 15u) != 0)
    return fail(kInvalidValue, "wna16_gemm: input must be 16-byte aligned");
  if (static_cast<long long>(size_m) * top_k > 0x7fffffffLL)
    return fail(kInvalidValue, "wna16_gemm: size_m * top_k overflows int32");
  if (cu_count <= 0) cu_count = current_cu_count();
  if (cu_count <= 0) return fail(kInvalidValue, "wna16_gemm: no device");

  const int max_m_blocks = ceil_div(sorted_token_ids_len, moe_block_size);
  const int n_tiles = size_n / 64;
  GemmArgs args{input, output, c_tmp, reinterpret_cast<const uint32_t*>(b_qweight), b_scales,
                workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
                sorted_token_ids_len, moe_block_size, top_k, mul_topk_weights ? 1 : 0, size_m,
                size_n, size_k, local_experts, 1};

  if (moe_block_size <= 16) {
    constexpr int WK = 4;
    const int groups = size_k / 32;
    const long long routes = static_cast<long long>(size_m) * top_k;
    const long long est_blocks = routes < max_m_blocks ? routes : max_m_blocks;
    const long long wgs = est_blocks * n_tiles;
    int splits = 1;
    const long long target = 2LL * cu_count;
    if (wgs < target) splits = static_cast<int>((target + wgs - 1) / wgs);
    const int max_split_by_k = groups / (WK * 2) > 0 ? groups / (WK * 2) : 1;
    if (splits > max_split_by_k) splits = max_split_by_k;
    // Partials need splits * sorted_len * N floats of c_tmp and one lock per
    // (m-block, tile); otherwise stay with one split.
    const long long per_split = static_cast<long long>(sorted_token_ids_len) * size_n;
    if (splits > 1) {
      long long cap = (c_tmp && per_split > 0) ? c_tmp_len / per_split : 0;
      if (!workspace || workspace_len < static_cast<long long>(max_m_blocks) * n_tiles) cap = 1;
      if (splits > cap) splits = cap < 1 ? 1 : static_cast<int>(cap);
    }
    args.splits = splits;
    const long long gx = static_cast<long long>(n_tiles) * splits;
    if (gx > 0x7fffffffLL || max_m_blocks > 65535)
      return fail(kNotSupported, "wna16_gemm: grid too large");
    hipLaunchKernelGGL(wna16_decode_kernel<WK>, dim3(static_cast<unsigned>(gx), max_m_blocks),
                       dim3(64 * WK), 0, stream, args);
    return launch_status("wna16_gemm (decode)");
  }
  if (max_m_blocks > 65535) return fail(kNotSupported, "wna16_gemm: too many m-blocks");
  hipLaunchKernelGGL(wna16_prefill_kernel, dim3(ceil_div(n_tiles, 4), max_m_blocks), dim3(256),
                     0, stream, args);
  return launch_status("wna16_gemm (prefill)");
}

}  // namespace pega

// ---------------------------------------------------------------- C ABI
// Reference: pegainfer-kernels/src/ffi/kimi.rs:131-152; launcher guards
// csrc/kimi_k2/kimi_marlin_wna16.cu:264-309 (local_experts == 48,
// group_size == 32, block size set, c_tmp required, workspace length).
// c_tmp is sized by the reference's convention (KimiMarlinWna16Workspace,
// src/ops/kimi_k2/experts.rs:612-652): size_n * sorted_token_ids_len floats,
// twice that for block size 8.  Locks are left at zero on return.
PEGA_API int kimi_marlin_wna16_gemm_cuda(
    const uint16_t* input, uint16_t* output, float* c_tmp, const uint8_t* b_qweight,
    const uint16_t* b_scales, int32_t* workspace, const int32_t* sorted_token_ids,
    const int32_t* expert_ids, const int32_t* num_tokens_post_padded, const float* topk_weights,
    int workspace_len, int sorted_token_ids_len, int moe_block_size, int top_k,
    bool mul_topk_weights, int size_m, int size_n, int size_k, int local_experts, int group_size,
    int sm_count, hipStream_t stream) {
  if (!workspace || !c_tmp)
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: workspace and c_tmp are required");
  if (local_experts != 48)
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: local_experts must be 48");
  if (size_k % 16 != 0 || size_n % 64 != 0 || size_k % group_size != 0)
    return pega::fail(pega::kInvalidValue, "kimi wna16_gemm: bad k/n");
  const long long c_tmp_len = static_cast<long long>(size_n) * sorted_token_ids_len *
                              (moe_block_size == 8 ? 2 : 1);
  return pega::wna16_gemm(input, output, c_tmp, c_tmp_len, b_qweight, b_scales, workspace,
                          workspace_len, sorted_token_ids, expert_ids, num_tokens_post_padded,
                          topk_weights, sorted_token_ids_len, moe_block_size, top_k,
                          mul_topk_weights, size_m, size_n, size_k, local_experts, group_size,
                          sm_count, stream);
}

// Shape-general entry (any expert count; explicit c_tmp length in floats and
// lock count; expert ids outside [0, local_experts) are skipped).  No
// reference counterpart: the reference accepts 48 experts only.
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
