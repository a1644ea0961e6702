/*
 * moe_oracle.c -- CPU restatement of PegaInfer's quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (pegainfer_amd) never calls it.
 *
 * Every function restates the scalar arithmetic of the reference file:line it
 * cites (paths relative to the reference repository root).  Build flags are
 * -O3 -ffp-contract=off so that every a*b+c below is two IEEE roundings unless
 * fmaf() is written explicitly (the reference uses an FMA there).
 *
 * Pinning (what checks each function independently of its own formula) is
 * listed per function; the tests live in tests/test_oracle.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                              */
/* ------------------------------------------------------------------------ */

static inline float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16 (the rounding __float2bfloat16 performs). */
static inline uint16_t to_bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint16_t oracle_f32_to_bf16(float f) { return to_bf(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf(h); }

/* exp used wherever the reference calls expf: the correctly rounded value of
 * e^x obtained from a double-precision exp.  The device code uses the same
 * definition for the router so that scores (and hence top-k indices) agree
 * bit for bit. */
static inline float exp_f32(float x) { return (float)exp((double)x); }
float oracle_expf(float x) { return exp_f32(x); }

/* ------------------------------------------------------------------------ */
/* K1: token -> expert permutation (kimi_moe_marlin_align_block_size)        */
/* pegainfer-kernels/csrc/kimi_k2/kimi_experts.cu:41-106 (single-block path,  */
/* whose order -- ascending route offset inside each expert -- is the one    */
/* the reference's KAT pins: pegainfer-kernels/src/ops/kimi_k2/experts.rs:    */
/* 1689-1717).  Pinned by: the KAT vector (tests/golden/align_kat.json), and  */
/* brute-force invariants on random inputs.                                  */
/* ------------------------------------------------------------------------ */
int oracle_align_block_size(const int32_t *topk_idx, int32_t *sorted_token_ids,
                            int32_t *expert_ids, int32_t *num_tokens_post_padded,
                            uint32_t *expert_offsets, uint32_t *expert_cursor,
                            int route_elems, int global_start, int local_experts,
                            int block_size, int max_padded_tokens, int max_m_blocks) {
  for (int i = 0; i < max_padded_tokens; ++i) sorted_token_ids[i] = route_elems;
  for (int i = 0; i < max_m_blocks; ++i) expert_ids[i] = -1;
  for (int e = 0; e <= local_experts; ++e) expert_offsets[e] = 0;
  for (int e = 0; e < local_experts; ++e) expert_cursor[e] = 0;
  /* histogram into offsets[e+1] (kimi_experts.cu:72-77) */
  for (int r = 0; r < route_elems; ++r) {
    int ex = topk_idx[r];
    if (ex >= global_start && ex < global_start + local_experts)
      expert_offsets[ex - global_start + 1] += 1u;
  }
  /* exclusive scan of padded counts, expert_ids per block (:82-94) */
  int total = 0;
  for (int e = 0; e < local_experts; ++e) {
    int count = (int)expert_offsets[e + 1];
    int padded = ((count + block_size - 1) / block_size) * block_size;
    expert_offsets[e] = (uint32_t)total;
    for (int pos = total; pos < total + padded; pos += block_size)
      expert_ids[pos / block_size] = e;
    total += padded;
  }
  expert_offsets[local_experts] = (uint32_t)total;
  num_tokens_post_padded[0] = total;
  /* stable scatter in route order (:96-105) */
  for (int r = 0; r < route_elems; ++r) {
    int ex = topk_idx[r];
    if (ex < global_start || ex >= global_start + local_experts) continue;
    int le = ex - global_start;
    int pos = (int)(expert_offsets[le] + expert_cursor[le]);
    expert_cursor[le] += 1u;
    if (pos < max_padded_tokens) sorted_token_ids[pos] = r;
  }
  return 0;
}

/* K9: routing metadata from an expert-major prefix sum
 * (kimi_experts.cu:372-433).  Identity ids over real rows, sentinel
 * max_padded_tokens over pad rows, expert_ids by the segment that holds the
 * block's first slot (0 past the total). */
int oracle_deepep_build_routing(const int32_t *psum_expert, int32_t *sorted_token_ids,
                                int32_t *expert_ids, int32_t *num_tokens_post_padded,
                                int num_local_experts, int alignment, int block_size,
                                int max_padded_tokens, int max_m_blocks) {
  int start[256], count[256];
  if (num_local_experts > 256) return 1;
  for (int e = 0; e < num_local_experts; ++e) {
    int s = 0;
    if (e > 0) s = ((psum_expert[e - 1] + alignment - 1) / alignment) * alignment;
    int c = psum_expert[e] - s;
    start[e] = s;
    count[e] = c < 0 ? 0 : c;
  }
  int total = psum_expert[num_local_experts];
  for (int idx = 0; idx < max_padded_tokens; ++idx) {
    int v = max_padded_tokens;
    if (idx < total) {
      int lo = 0;
      for (int e = 0; e < num_local_experts; ++e)
        if (start[e] <= idx) lo = e; /* largest e with start<=idx (starts non-decreasing) */
      if (idx - start[lo] < count[lo]) v = idx;
    }
    sorted_token_ids[idx] = v;
  }
  for (int b = 0; b < max_m_blocks; ++b) {
    int slot = b * block_size, ex = 0;
    if (slot < total) {
      for (int e = 0; e < num_local_experts; ++e)
        if (start[e] <= slot) ex = e;
    }
    expert_ids[b] = ex;
  }
  num_tokens_post_padded[0] = total;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* K5/K6/K7: Marlin layout repacks                                           */
/* ------------------------------------------------------------------------ */

/* K5 (kimi_marlin_int4.cu:21-96).  Written as the direct index map of the
 * reference kernel: output word (k_tile, n_tile, th, w) of a 16x64 tile packs
 * the 8 nibbles (n, k) with
 *     n  = n_tile*64 + w*16 + th/4 + {0, 8}
 *     k  = k_tile*16 + 2*(th%4) + {0, 1, 8, 9}
 * in nibble order pack_idx = {0,2,4,6,1,3,5,7} over
 *     vals = {(n,k0),(n,k1),(n,k8),(n,k9),(n+8,k0),(n+8,k1),(n+8,k8),(n+8,k9)}.
 * Checkpoint words are [E][N][K/8] with element k%8 at bits 4*(k%8).
 * Pinned by: the reference's KAT builder restated in tests/golden
 * (experts.rs:1798-1878), and the inverse map oracle_marlin_unpack_weight. */
static inline uint32_t ckpt_nibble(const uint32_t *ck, int k_words, int n, int k) {
  return (ck[(size_t)n * k_words + (k >> 3)] >> ((k & 7) * 4)) & 0xfu;
}

int oracle_marlin_reorder_weight(const uint32_t *ckpt, uint32_t *marlin, int in_dim,
                                 int out_dim, int local_experts) {
  if (in_dim % 16 || out_dim % 64) return 1;
  const int k_words = in_dim / 8, k_tiles = in_dim / 16, n_tiles = out_dim / 64;
  const size_t per_expert = (size_t)out_dim * k_words;
  static const int koff[4] = {0, 1, 8, 9};
  static const int pack_idx[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  for (int e = 0; e < local_experts; ++e) {
    const uint32_t *ck = ckpt + e * per_expert;
    uint32_t *mw = marlin + e * per_expert;
    for (int kt = 0; kt < k_tiles; ++kt)
      for (int nt = 0; nt < n_tiles; ++nt)
        for (int th = 0; th < 32; ++th)
          for (int w = 0; w < 4; ++w) {
            int n = nt * 64 + w * 16 + th / 4;
            int kb = kt * 16 + 2 * (th % 4);
            uint32_t vals[8];
            for (int i = 0; i < 4; ++i) {
              vals[i] = ckpt_nibble(ck, k_words, n, kb + koff[i]);
              vals[4 + i] = ckpt_nibble(ck, k_words, n + 8, kb + koff[i]);
            }
            uint32_t res = 0;
            for (int i = 0; i < 8; ++i) res |= vals[pack_idx[i]] << (i * 4);
            mw[((size_t)kt * n_tiles + nt) * 128 + th * 4 + w] = res;
          }
  }
  return 0;
}

/* Inverse of K5: Marlin words back to checkpoint words (used to prove the
 * repack is a bijection on nibbles). */
int oracle_marlin_unpack_weight(const uint32_t *marlin, uint32_t *ckpt, int in_dim,
                                int out_dim, int local_experts) {
  if (in_dim % 16 || out_dim % 64) return 1;
  const int k_words = in_dim / 8, k_tiles = in_dim / 16, n_tiles = out_dim / 64;
  const size_t per_expert = (size_t)out_dim * k_words;
  /* nibble slot i of a Marlin word -> (dn, dk) */
  static const int slot_dn[8] = {0, 0, 8, 8, 0, 0, 8, 8};
  static const int slot_dk[8] = {0, 8, 0, 8, 1, 9, 1, 9};
  memset(ckpt, 0, sizeof(uint32_t) * per_expert * local_experts);
  for (int e = 0; e < local_experts; ++e) {
    const uint32_t *mw = marlin + e * per_expert;
    uint32_t *ck = ckpt + e * per_expert;
    for (int kt = 0; kt < k_tiles; ++kt)
      for (int nt = 0; nt < n_tiles; ++nt)
        for (int th = 0; th < 32; ++th)
          for (int w = 0; w < 4; ++w) {
            uint32_t word = mw[((size_t)kt * n_tiles + nt) * 128 + th * 4 + w];
            int n = nt * 64 + w * 16 + th / 4;
            int kb = kt * 16 + 2 * (th % 4);
            for (int i = 0; i < 8; ++i) {
              int nn = n + slot_dn[i], kk = kb + slot_dk[i];
              uint32_t v = (word >> (4 * i)) & 0xfu;
              ck[(size_t)nn * k_words + (kk >> 3)] |= v << ((kk & 7) * 4);
            }
          }
  }
  return 0;
}

/* K6 (kimi_marlin_int4.cu:119-142): [E][N][K/32] -> [E][K/32][N] with each
 * 64-element chunk permuted by p(o) = o/8 + 8*(o%8).
 * Pinned by: the reference's KAT (experts.rs:1730-1796) restated in
 * tests/golden. */
int oracle_marlin_reorder_scale(const uint16_t *ckpt, uint16_t *marlin, int in_dim,
                                int out_dim, int local_experts, int group_size) {
  if (in_dim % group_size) return 1;
  const int scale_k = in_dim / group_size;
  const size_t per_expert = (size_t)out_dim * scale_k;
  if (per_expert % 64) return 1;
  for (int e = 0; e < local_experts; ++e)
    for (size_t idx = 0; idx < per_expert; ++idx) {
      size_t chunk = idx / 64;
      int o = (int)(idx % 64);
      size_t t = chunk * 64 + (size_t)(o / 8 + 8 * (o % 8));
      int g = (int)(t / out_dim);
      int row = (int)(t - (size_t)g * out_dim);
      marlin[e * per_expert + idx] = ckpt[e * per_expert + (size_t)row * scale_k + g];
    }
  return 0;
}

/* K7 (kimi_marlin_int4.cu:98-117,144-163): per (expert, k-tile) row, gate words
 * then up words; per (expert, group) row, gate scales then up scales. */
int oracle_marlin_fuse_w13(const uint32_t *gate_w, const uint32_t *up_w, uint32_t *w13_w,
                           const uint16_t *gate_s, const uint16_t *up_s, uint16_t *w13_s,
                           int in_dim, int inter, int local_experts, int group_size) {
  const size_t rows_w = (size_t)local_experts * (in_dim / 16);
  const size_t cols_w = (size_t)inter * 2;
  for (size_t r = 0; r < rows_w; ++r) {
    memcpy(w13_w + r * 2 * cols_w, gate_w + r * cols_w, cols_w * 4);
    memcpy(w13_w + r * 2 * cols_w + cols_w, up_w + r * cols_w, cols_w * 4);
  }
  const size_t rows_s = (size_t)local_experts * (in_dim / group_size);
  const size_t cols_s = (size_t)inter;
  for (size_t r = 0; r < rows_s; ++r) {
    memcpy(w13_s + r * 2 * cols_s, gate_s + r * cols_s, cols_s * 2);
    memcpy(w13_s + r * 2 * cols_s + cols_s, up_s + r * cols_s, cols_s * 2);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* K2: grouped W4A16 GEMM semantics                                          */
/* marlin_template.h:112-124 (w = bf16(q*s), __hmul2 in bf16),               */
/*   :466-537 (row mapping, topk weight rounded to bf16),                    */
/*   :1411-1426 (bf16 x bf16 MMA, fp32 accumulate),                          */
/*   :1806-1807, 1878-1890 (bf16(acc), optional bf16(c*bf16(w)), skip rows). */
/* The oracle takes checkpoint-layout weights ([E][N][K/2] bytes, low nibble  */
/* = even column; scales [E][N][K/groups]) so that it shares no code with the */
/* Marlin layout the device consumes.  Accumulation is sequential in k, in    */
/* fp32 (the reference's tensor-core order is not reproducible; the          */
/* tolerance covers order).  Pinned by exact special cases (power-of-two     */
/* scales, small-integer activations => every partial sum exact), one-hot     */
/* rows, zero weights, and an fp64 brute force with an error bound.          */
/* ------------------------------------------------------------------------ */

typedef struct {
  const uint16_t *input;
  uint16_t *output;
  const uint8_t *qweight; /* checkpoint [E][N][K/2] */
  const uint16_t *scales; /* checkpoint [E][N][K/group] */
  const int32_t *sorted_token_ids;
  const int32_t *expert_ids;
  const int32_t *num_tokens_post_padded;
  const float *topk_weights;
  int moe_block_size, top_k, mul_topk_weights, size_m, size_n, size_k, group_size;
  int n_items;            /* (m-block, n-chunk) work items */
  int n_chunk;            /* columns per work item */
  volatile int next_item; /* shared work counter */
  pthread_mutex_t lock;
} gemm_job;

static void gemm_block(gemm_job *j, int mb, int n0, int n1, float *wrow) {
  const int K = j->size_k, G = j->group_size, kg = K / G;
  const int ntp = j->num_tokens_post_padded[0];
  if (mb * j->moe_block_size >= ntp) return;
  int ex = j->expert_ids[mb];
  if (ex < 0) return;
  const size_t e_w = (size_t)j->size_n * (K / 2), e_s = (size_t)j->size_n * kg;
  const int valid_limit = j->size_m * j->top_k;
  for (int n = n0; n < n1; ++n) {
    const uint8_t *qrow = j->qweight + ex * e_w + (size_t)n * (K / 2);
    const uint16_t *srow = j->scales + ex * e_s + (size_t)n * kg;
    /* dequantised column n: w = bf16((nibble - 8) * s) */
    for (int k = 0; k < K; ++k) {
      uint8_t byte = qrow[k >> 1];
      int nib = (k & 1) ? (byte >> 4) : (byte & 0xf);
      float s = bf(srow[k / G]);
      wrow[k] = bf(to_bf((float)(nib - 8) * s));
    }
    for (int i = 0; i < j->moe_block_size; ++i) {
      int sid = j->sorted_token_ids[mb * j->moe_block_size + i];
      if (sid >= valid_limit) continue;
      const uint16_t *a = j->input + (size_t)(sid / j->top_k) * K;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc += bf(a[k]) * wrow[k];
      uint16_t c = to_bf(acc);
      if (j->mul_topk_weights) {
        float tw = bf(to_bf(j->topk_weights[sid]));
        c = to_bf(bf(c) * tw);
      }
      j->output[(size_t)sid * j->size_n + n] = c;
    }
  }
}

static void *gemm_worker(void *arg) {
  gemm_job *j = (gemm_job *)arg;
  float *wrow = (float *)malloc(sizeof(float) * (size_t)j->size_k);
  const int n_chunks = (j->size_n + j->n_chunk - 1) / j->n_chunk;
  for (;;) {
    pthread_mutex_lock(&j->lock);
    int item = j->next_item++;
    pthread_mutex_unlock(&j->lock);
    if (item >= j->n_items) break;
    int mb = item / n_chunks, nc = item % n_chunks;
    int n0 = nc * j->n_chunk, n1 = n0 + j->n_chunk;
    if (n1 > j->size_n) n1 = j->size_n;
    gemm_block(j, mb, n0, n1, wrow);
  }
  free(wrow);
  return NULL;
}

int oracle_wna16_gemm(const uint16_t *input, uint16_t *output, const uint8_t *qweight,
                      const uint16_t *scales, const int32_t *sorted_token_ids,
                      const int32_t *expert_ids, const int32_t *num_tokens_post_padded,
                      const float *topk_weights, int max_m_blocks, int moe_block_size,
                      int top_k, int mul_topk_weights, int size_m, int size_n, int size_k,
                      int group_size, int threads) {
  if (size_k % group_size || size_k % 2) return 1;
  gemm_job j;
  memset(&j, 0, sizeof(j));
  j.input = input; j.output = output; j.qweight = qweight; j.scales = scales;
  j.sorted_token_ids = sorted_token_ids; j.expert_ids = expert_ids;
  j.num_tokens_post_padded = num_tokens_post_padded; j.topk_weights = topk_weights;
  j.moe_block_size = moe_block_size; j.top_k = top_k; j.mul_topk_weights = mul_topk_weights;
  j.size_m = size_m; j.size_n = size_n; j.size_k = size_k; j.group_size = group_size;
  j.n_chunk = 64;
  j.n_items = max_m_blocks * ((size_n + j.n_chunk - 1) / j.n_chunk);
  pthread_mutex_init(&j.lock, NULL);
  if (threads < 1) threads = 1;
  if (threads == 1) {
    gemm_worker(&j);
  } else {
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    for (int t = 0; t < threads; ++t) pthread_create(&tid[t], NULL, gemm_worker, &j);
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(tid);
  }
  pthread_mutex_destroy(&j.lock);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* CPU BASELINE ONLY (bench.py's cpu_baseline leg), not a checker: the same  */
/* grouped GEMM contract as oracle_wna16_gemm (dequant w = bf16((q-8)*s),     */
/* fp32 products, bf16 output, bf16 top-k weight multiply) with the fp32 sum */
/* of each output split into 16 lane sums that are added in a fixed tree     */
/* order at the end, so the compiler can vectorise the dot products and the  */
/* dequant.  target_clones builds AVX-512, AVX2 and baseline versions, picked */
/* at load time for the host CPU.  Checked against oracle_wna16_gemm (bit   */
/* for bit where every partial sum is exact, within the fp32 bound           */
/* otherwise) in tests/test_oracle.py.                                       */
/* ------------------------------------------------------------------------ */
#define CLONES __attribute__((target_clones("avx512f", "avx2", "default")))

CLONES static void dequant_col_fast(const uint8_t *q, const uint16_t *sc, int K, int G,
                                    float *w) {
  for (int g = 0; g < K / G; ++g) {
    const float s = bf(sc[g]);
    const uint8_t *qg = q + (size_t)g * (G / 2);
    float *wg = w + (size_t)g * G;
    for (int j = 0; j < G / 2; ++j) {
      const float lo = (float)((int)(qg[j] & 15) - 8) * s;
      const float hi = (float)((int)(qg[j] >> 4) - 8) * s;
      uint32_t ul, uh;
      memcpy(&ul, &lo, 4);
      memcpy(&uh, &hi, 4);
      ul = (ul + 0x7fffu + ((ul >> 16) & 1u)) & 0xffff0000u; /* finite: no NaN case */
      uh = (uh + 0x7fffu + ((uh >> 16) & 1u)) & 0xffff0000u;
      memcpy(&wg[2 * j], &ul, 4);
      memcpy(&wg[2 * j + 1], &uh, 4);
    }
  }
}

CLONES static float dot16(const float *a, const float *w, int K) {
  float acc[16] = {0};
  int k = 0;
  for (; k + 16 <= K; k += 16)
    for (int j = 0; j < 16; ++j) acc[j] += a[k + j] * w[k + j];
  for (; k < K; ++k) acc[k & 15] += a[k] * w[k];
  for (int st = 8; st > 0; st >>= 1)
    for (int j = 0; j < st; ++j) acc[j] += acc[j + st];
  return acc[0];
}

static void gemm_block_fast(gemm_job *j, int mb, int n0, int n1, float *wcol, float *arows) {
  const int K = j->size_k, G = j->group_size, kg = K / G;
  const int ntp = j->num_tokens_post_padded[0];
  if (mb * j->moe_block_size >= ntp) return;
  int ex = j->expert_ids[mb];
  if (ex < 0) return;
  const size_t e_w = (size_t)j->size_n * (K / 2), e_s = (size_t)j->size_n * kg;
  const int valid_limit = j->size_m * j->top_k;
  int sids[64], nrows = 0;
  for (int i = 0; i < j->moe_block_size && i < 64; ++i) {
    int sid = j->sorted_token_ids[mb * j->moe_block_size + i];
    if (sid >= valid_limit) continue;
    const uint16_t *a = j->input + (size_t)(sid / j->top_k) * K;
    float *ar = arows + (size_t)nrows * K;
    for (int k = 0; k < K; ++k) ar[k] = bf(a[k]);
    sids[nrows++] = sid;
  }
  if (nrows == 0) return;
  for (int n = n0; n < n1; ++n) {
    dequant_col_fast(j->qweight + ex * e_w + (size_t)n * (K / 2), j->scales + ex * e_s +
                     (size_t)n * kg, K, G, wcol);
    for (int r = 0; r < nrows; ++r) {
      uint16_t c = to_bf(dot16(arows + (size_t)r * K, wcol, K));
      if (j->mul_topk_weights) c = to_bf(bf(c) * bf(to_bf(j->topk_weights[sids[r]])));
      j->output[(size_t)sids[r] * j->size_n + n] = c;
    }
  }
}

static void *gemm_worker_fast(void *arg) {
  gemm_job *j = (gemm_job *)arg;
  float *wcol = (float *)malloc(sizeof(float) * (size_t)j->size_k);
  float *arows = (float *)malloc(sizeof(float) * (size_t)j->size_k * 64);
  const int n_chunks = (j->size_n + j->n_chunk - 1) / j->n_chunk;
  for (;;) {
    pthread_mutex_lock(&j->lock);
    int item = j->next_item++;
    pthread_mutex_unlock(&j->lock);
    if (item >= j->n_items) break;
    int mb = item / n_chunks, nc = item % n_chunks;
    int n0 = nc * j->n_chunk, n1 = n0 + j->n_chunk;
    if (n1 > j->size_n) n1 = j->size_n;
    gemm_block_fast(j, mb, n0, n1, wcol, arows);
  }
  free(wcol);
  free(arows);
  return NULL;
}

int oracle_wna16_gemm_fast(const uint16_t *input, uint16_t *output, const uint8_t *qweight,
                           const uint16_t *scales, const int32_t *sorted_token_ids,
                           const int32_t *expert_ids, const int32_t *num_tokens_post_padded,
                           const float *topk_weights, int max_m_blocks, int moe_block_size,
                           int top_k, int mul_topk_weights, int size_m, int size_n, int size_k,
                           int group_size, int threads) {
  if (size_k % group_size || size_k % 2 || group_size % 2 || moe_block_size > 64) return 1;
  gemm_job j;
  memset(&j, 0, sizeof(j));
  j.input = input; j.output = output; j.qweight = qweight; j.scales = scales;
  j.sorted_token_ids = sorted_token_ids; j.expert_ids = expert_ids;
  j.num_tokens_post_padded = num_tokens_post_padded; j.topk_weights = topk_weights;
  j.moe_block_size = moe_block_size; j.top_k = top_k; j.mul_topk_weights = mul_topk_weights;
  j.size_m = size_m; j.size_n = size_n; j.size_k = size_k; j.group_size = group_size;
  j.n_chunk = 64;
  j.n_items = max_m_blocks * ((size_n + j.n_chunk - 1) / j.n_chunk);
  pthread_mutex_init(&j.lock, NULL);
  if (threads < 1) threads = 1;
  if (threads == 1) {
    gemm_worker_fast(&j);
  } else {
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    for (int t = 0; t < threads; ++t) pthread_create(&tid[t], NULL, gemm_worker_fast, &j);
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(tid);
  }
  pthread_mutex_destroy(&j.lock);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* K3: SwiGLU (kimi_marlin_wna16.cu:345-361):                                */
/*   out = bf16( f(bf16( g/(1+exp(-g)) )) * u ),  g = w13[r,c], u = w13[r,I+c] */
/* Pinned by: fp64 evaluation of the same closed form (agreement to 1 bf16   */
/* ulp only where the fp32 silu sits on a bf16 rounding tie), g = 0, and      */
/* saturation limits.                                                         */
/* ------------------------------------------------------------------------ */
int oracle_swiglu(const uint16_t *w13, uint16_t *out, int rows, int inter) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < inter; ++c) {
      float g = bf(w13[(size_t)r * 2 * inter + c]);
      float u = bf(w13[(size_t)r * 2 * inter + inter + c]);
      float silu = g / (1.0f + exp_f32(-g));
      out[(size_t)r * inter + c] = to_bf(bf(to_bf(silu)) * u);
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Dense bf16 GEMM of the shared expert (pegainfer-kernels/csrc/shared/      */
/* linear.cu:321-344, gemm_graphsafe_cuda: cublasGemmEx(OP_T, OP_N, M, N, K,  */
/* W lda K, X ldb K, Y ldc M, CUBLAS_COMPUTE_32F), called from               */
/* pegainfer-kimi-k2/src/runner/moe_nccl.rs:107-123):                         */
/*   Y[n][m] = bf16( sum_k f(W[m][k]) * f(X[n][k]) ),  fp32 accumulation     */
/* (k ascending here; the library's order is its own, so parity is to the    */
/* tolerance).  W [M][K], X [N][K], Y [N][M], all bf16 row-major.            */
/* Pinned by: small-integer operands with power-of-two scales (every partial */
/* sum exact, so any order gives these bits), one-hot rows of X (Y equals a  */
/* column of W), zero W, and fp64 brute force on random operands within the */
/* fp32-accumulation bound.                                                 */
/* ------------------------------------------------------------------------ */
int oracle_dense_gemm(const uint16_t *W, const uint16_t *X, uint16_t *Y, int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  float *wrow = (float *)malloc(sizeof(float) * (size_t)K);
  float *xrow = (float *)malloc(sizeof(float) * (size_t)K);
  if (!wrow || !xrow) {
    free(wrow);
    free(xrow);
    return 2;
  }
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) xrow[k] = bf(X[(size_t)n * K + k]);
    for (int m = 0; m < M; ++m) {
      for (int k = 0; k < K; ++k) wrow[k] = bf(W[(size_t)m * K + k]);
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc += wrow[k] * xrow[k];
      Y[(size_t)n * M + m] = to_bf(acc);
    }
  }
  free(wrow);
  free(xrow);
  return 0;
}

/* Router logits GEMM of kimi_k2_router_noaux_tc (pegainfer-kernels/csrc/kimi_k2/      */
/* kimi_router.cu:108-142: cublasGemmEx(OP_T, OP_N, n_experts, padded_tokens,         */
/* hidden_dim, gate lda hidden_dim, hidden ldb hidden_dim, logits CUDA_R_32F ldc       */
/* n_experts, CUBLAS_COMPUTE_32F_PEDANTIC)):                                          */
/*   Y[n][m] = sum_k f(W[m][k]) * f(X[n][k])  in fp32, NOT rounded to bf16            */
/* (k ascending here; parity to the fp32-accumulation bound).  Pinned by: small-      */
/* integer operands whose every partial sum is exact (any order gives these bits),   */
/* one-hot rows of X (Y is a row of W exactly), bf16(Y) == oracle_dense_gemm, and an  */
/* fp64 bound on random operands.                                                    */
int oracle_dense_gemm_f32(const uint16_t *W, const uint16_t *X, float *Y, int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  float *xrow = (float *)malloc(sizeof(float) * (size_t)K);
  if (!xrow) return 2;
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) xrow[k] = bf(X[(size_t)n * K + k]);
    for (int m = 0; m < M; ++m) {
      const uint16_t *w = W + (size_t)m * K;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc += bf(w[k]) * xrow[k];
      Y[(size_t)n * M + m] = acc;
    }
  }
  free(xrow);
  return 0;
}

/* f32_to_bf16_cuda (pegainfer-kernels/csrc/shared/elementwise.cu:235-244):           */
/* out = bf16(x), round to nearest even.  Pinned by: numpy's independent rounding     */
/* (tests) and the tie cases 1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6.                    */
int oracle_f32_to_bf16_n(const float *x, uint16_t *out, int n) {
  for (int i = 0; i < n; ++i) out[i] = to_bf(x[i]);
  return 0;
}

/* add_cuda / add_kernel (pegainfer-kernels/csrc/shared/elementwise.cu:9-21):          */
/* out = bf16(f(a) + f(b)).  With oracle_f32_to_bf16_n first it is the DeepSeek-V2-   */
/* Lite routed + shared join (nccl_backend.rs:544-545, runtime/moe.rs:656).  Pinned  */
/* by: numpy float32 addition and rounding, and inputs on which the join's two        */
/* roundings differ from one rounding of routed + shared.                             */
int oracle_add_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, int n) {
  for (int i = 0; i < n; ++i) out[i] = to_bf(bf(a[i]) + bf(b[i]));
  return 0;
}

/* K4: top-k row sum (kimi_marlin_wna16.cu:392-408): fp32, k ascending from 0.
 * Pinned by: numpy float32 sequential accumulation. */
int oracle_sum_topk_rows(const uint16_t *route_output, float *out, int active_tokens,
                         int topk, int hidden) {
  for (int t = 0; t < active_tokens; ++t)
    for (int d = 0; d < hidden; ++d) {
      float acc = 0.0f;
      for (int k = 0; k < topk; ++k) acc += bf(route_output[((size_t)t * topk + k) * hidden + d]);
      out[(size_t)t * hidden + d] = acc;
    }
  return 0;
}

/* K8 (kimi_experts.cu:25-39, 308-322) and K10 (:15-23). */
int oracle_residual_add_scaled_f32(const uint16_t *hidden, const uint16_t *projected,
                                   const float *routed, float scale, uint16_t *out, int n) {
  for (int i = 0; i < n; ++i) {
    uint16_t rounded = to_bf(bf(hidden[i]) + bf(projected[i]));
    float scaled = routed[i] * scale;
    out[i] = to_bf(scaled + bf(rounded));
  }
  return 0;
}

int oracle_residual_add_scaled_bf16(const uint16_t *hidden, const uint16_t *projected,
                                    const uint16_t *routed, float scale, uint16_t *out,
                                    int n) {
  for (int i = 0; i < n; ++i) {
    uint16_t rounded = to_bf(bf(hidden[i]) + bf(projected[i]));
    float scaled = bf(routed[i]) * scale;
    out[i] = to_bf(scaled + bf(rounded));
  }
  return 0;
}

int oracle_add_f32_bf16(const float *a, const uint16_t *b, uint16_t *out, int n) {
  for (int i = 0; i < n; ++i) out[i] = to_bf(a[i] + bf(b[i]));
  return 0;
}

/* ------------------------------------------------------------------------ */
/* R1: Kimi noaux_tc router select (kimi_router.cu:20-91; route_scale 1.0,    */
/* router.rs:19,39).  score = 1/(1+exp(-l)); pick topk by score+bias         */
/* descending, ties -> lower id, kept in selection order; weight =           */
/* score * (route_scale / sum), sum accumulated in selection order.          */
/* Pinned by: brute-force stable sort on random logits.                      */
/* ------------------------------------------------------------------------ */
int oracle_kimi_router(const float *logits, const float *bias, float *topk_weight,
                       int32_t *topk_idx, int tokens, int n_experts, int topk,
                       float route_scale) {
  float *score = (float *)malloc(sizeof(float) * n_experts);
  float *choice = (float *)malloc(sizeof(float) * n_experts);
  for (int t = 0; t < tokens; ++t) {
    for (int e = 0; e < n_experts; ++e) {
      score[e] = 1.0f / (1.0f + exp_f32(-logits[(size_t)t * n_experts + e]));
      choice[e] = score[e] + bias[e];
    }
    float sel[64];
    float sum = 0.0f;
    for (int r = 0; r < topk; ++r) {
      int best = n_experts;
      float bv = -INFINITY;
      for (int e = 0; e < n_experts; ++e)
        if (choice[e] > bv || (choice[e] == bv && e < best)) { bv = choice[e]; best = e; }
      float s = best < n_experts ? score[best] : 0.0f;
      sel[r] = s;
      topk_idx[t * topk + r] = best;
      sum += s;
      if (best < n_experts) choice[best] = -INFINITY;
    }
    float scale = sum > 0.0f ? route_scale / sum : 0.0f;
    for (int r = 0; r < topk; ++r) topk_weight[t * topk + r] = sel[r] * scale;
  }
  free(score);
  free(choice);
  return 0;
}

/* R2: DSV2-Lite softmax top-k (pegainfer-deepseek-v2-lite/src/host_ops.rs:
 * 388-412, 431-445): probs = exp(l - max) / sum (sum sequential), take topk by
 * prob descending (ties -> lower id), then order the selection by expert id;
 * weight = prob (norm_topk_prob=false, routed_scaling_factor=1.0).
 * Pinned by: the reference's test (host_ops.rs:536-554) and brute force. */
int oracle_dsv2_router(const float *logits, float *topk_weight, int32_t *topk_idx,
                       int tokens, int n_experts, int topk) {
  float *p = (float *)malloc(sizeof(float) * n_experts);
  char *taken = (char *)malloc(n_experts);
  for (int t = 0; t < tokens; ++t) {
    const float *l = logits + (size_t)t * n_experts;
    float mx = -INFINITY;
    for (int e = 0; e < n_experts; ++e) mx = l[e] > mx ? l[e] : mx;
    float sum = 0.0f;
    for (int e = 0; e < n_experts; ++e) { p[e] = exp_f32(l[e] - mx); sum += p[e]; }
    for (int e = 0; e < n_experts; ++e) p[e] = sum == 0.0f ? 0.0f : p[e] / sum;
    memset(taken, 0, n_experts);
    int idx[64];
    for (int r = 0; r < topk; ++r) {
      int best = -1;
      for (int e = 0; e < n_experts; ++e) {
        if (taken[e]) continue;
        if (best < 0 || p[e] > p[best]) best = e;
      }
      taken[best] = 1;
      idx[r] = best;
    }
    /* insertion sort by id */
    for (int i = 1; i < topk; ++i) {
      int v = idx[i], j = i - 1;
      while (j >= 0 && idx[j] > v) { idx[j + 1] = idx[j]; --j; }
      idx[j + 1] = v;
    }
    for (int r = 0; r < topk; ++r) {
      topk_idx[t * topk + r] = idx[r];
      topk_weight[t * topk + r] = p[idx[r]];
    }
  }
  free(p);
  free(taken);
  return 0;
}

/* Weighted fp32 accumulate of routed rows in route-plan order
 * (accumulate_fixed_expert_kernel, dsv2_lite_moe.cu:131-155, explicit fmaf):
 *   out[t,d] = fma(f(route_out[t*topk+k, d]), w[t,k], out[t,d])  for k ascending. */
int oracle_weighted_topk_sum(const uint16_t *route_output, const float *topk_weight,
                             float *out, int tokens, int topk, int hidden) {
  for (int t = 0; t < tokens; ++t)
    for (int d = 0; d < hidden; ++d) {
      float acc = 0.0f;
      for (int k = 0; k < topk; ++k)
        acc = fmaf(bf(route_output[((size_t)t * topk + k) * hidden + d]),
                   topk_weight[t * topk + k], acc);
      out[(size_t)t * hidden + d] = acc;
    }
  return 0;
}
