// Dense bf16 GEMM of the shared expert on MI355X (gfx950):
//
//   Y[n][m] = bf16( sum_k f(W[m][k]) * f(X[n][k]) ),  fp32 accumulation,
//   W [M][K], X [N][K], Y [N][M], bf16 row-major
//
// Reference: pegainfer-kernels/csrc/shared/linear.cu:321-344
// (gemm_graphsafe_cuda: cublasGemmEx(OP_T, OP_N, M, N, K, W lda K, X ldb K,
// Y ldc M, CUBLAS_COMPUTE_32F)), bound in pegainfer-kernels/src/ffi/shared.rs:220-238
// and called for the Kimi shared expert's gate/up and down projections
// (pegainfer-kimi-k2/src/runner/moe_nccl.rs:107-123).
//
// Load shape: the 16x16x32 fragment layout puts a different W (or X) row in
// each of four neighbouring lanes; loaded that way, every 16-byte-per-lane
// load splits into about 64 cache-line requests and the address unit bounds
// the kernel (78% busy, ~77 cycles per load instruction, 1.6 TB/s of W on the
// Kimi gate/up shape).  So the loads run along k (a lane quad reads 64
// contiguous bytes of one row) and ds_bpermute moves each lane's 16 bytes to
// the lane whose fragment needs them: gate/up 37.3 -> 26.4 us (2.3 TB/s of W).
// A permuted k order that reads 256 contiguous bytes per row per step instead
// quadruples the lines per instruction and ran 2.3x slower.
//
// The decode-sized token counts this serves make the GEMM a weight stream:
// one workgroup owns 16 MR output features for 16 RB tokens (the host picks
// the shape); its WK waves split K and are reduced through LDS in wave order
// (deterministic).  Per 32-k step a lane issues one 16-byte load of W per
// 16-feature row tile and one of X per 16-token row block; after the lane
// exchange, lane (c, q) holds feature m0 + 16 mr + c, k 8q..8q+7 (the B
// fragment of a 16x16x32 MFMA) and the token blocks' A fragments, and one
// v_mfma_f32_16x16x32_bf16 runs per (row tile, token block).  A and B take
// the same k slots per lane, so the product is exact whatever k order the
// MFMA assigns to them.  Token rows past N read zeros through an
// out-of-range buffer offset and are never stored.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

constexpr uint32_t kOutOfRange = 0x80000000u;  // voffset that fails every range check
// W loads are cached too: a step reads 64 bytes of each of 16 rows, so the
// other half of every 128-byte line is the next step's, and a non-temporal
// policy that does not keep the line costs 20% (44.9 against 37.3 us for
// the Kimi gate/up shape).
constexpr int kCached = 0;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

template <int kPolicy>
__device__ __forceinline__ u32x4_t load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff),
                                               kPolicy);
}

template <int MR, int RB>
struct StepRegs {
  u32x4_t w[MR];  // W[m0 + 16 mr + l / 4][k0 + 8 (l % 4) .. +7] (lane l)
  u32x4_t x[RB];  // X[n0 + 16 rb + l / 4][k0 + 8 (l % 4) .. +7]
};

// One workgroup per (16 MR output features, 16 RB tokens); WK waves split the
// K/32 steps; D steps per wave in flight.  Each X fragment feeds MR MFMAs and
// each W fragment RB.  A wave's row tiles start tile_stride rows apart.
// SWIGLU (MR = 2): tile 0 holds gate features m0..m0+15 and tile 1 the
// matching up features (tile_stride = I); the epilogue rounds both sums to
// bf16 as the GEMM's output would be, applies SwiGLU and writes act[n][m0+c]
// (Y row stride M = I).  F32: Y is fp32 and takes the sums unrounded (the
// router's logits GEMM, cublasGemmEx with CUDA_R_32F output).
template <int WK, int MR, int RB, bool SWIGLU, bool F32 = false>
__global__ __launch_bounds__(64 * WK) void dense_gemm_kernel(const uint16_t* __restrict__ W,
                                                             const uint16_t* __restrict__ X,
                                                             void* __restrict__ Yv, int M,
                                                             int N, int K, int tile_stride) {
  static_assert(!SWIGLU || MR == 2, "SwiGLU pairs one gate and one up tile");
  static_assert(!(SWIGLU && F32), "the SwiGLU epilogue writes bf16");
  uint16_t* __restrict__ Y = static_cast<uint16_t*>(Yv);
  constexpr int D = MR + RB <= 5 ? 4 : 3;  // the ring fits 128 VGPRs at WK = 16
  __shared__ float s_red[WK][RB * 4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.x * (SWIGLU ? 16 : 16 * MR);
  const int n0 = blockIdx.y * (16 * RB);
  const int steps = K >> 5;
  const int s0 = (steps * wave) / WK, s1 = (steps * (wave + 1)) / WK;

  const __amdgpu_buffer_rsrc_t wr = make_rsrc(
      W + static_cast<long long>(m0) * K,
      (static_cast<uint32_t>(tile_stride) * (MR - 1) + 16u) * static_cast<uint32_t>(K) * 2u);
  // Loads run along k: lane l fetches row l / 4, k 8 (l % 4) .. +7, so four
  // neighbouring lanes read 64 contiguous bytes of one row (one line request
  // per lane quad, 16 per load); ds_bpermute then hands lane (c, q) the
  // 16 bytes of row c, k 8q .. +7 that its fragment needs, from lane 4c + q.
  const uint32_t lr = static_cast<uint32_t>(lane >> 2), lp = static_cast<uint32_t>(lane & 3);
  uint32_t w_voff[MR];
#pragma unroll
  for (int mr = 0; mr < MR; ++mr) w_voff[mr] = ((static_cast<uint32_t>(tile_stride) * mr + lr) * K + 8u * lp) * 2u;
  const int src_lane_bytes = (4 * c + q) * 4;
  const __amdgpu_buffer_rsrc_t xr =
      make_rsrc(X, static_cast<uint32_t>(N) * static_cast<uint32_t>(K) * 2u);
  uint32_t x_voff[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int n = n0 + 16 * rb + static_cast<int>(lr);
    x_voff[rb] = n < N ? (static_cast<uint32_t>(n) * K + 8u * lp) * 2u : kOutOfRange;
  }
  auto to_fragment = [&](u32x4_t v) {
    u32x4_t f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      f[e] = static_cast<uint32_t>(
          __builtin_amdgcn_ds_bpermute(src_lane_bytes, static_cast<int>(v[e])));
    return __builtin_bit_cast(bf16x8_t, f);
  };

  auto load_step = [&](StepRegs<MR, RB>& r, int s) {
    s = min(max(s, 0), steps - 1);  // every scalar offset stays inside the rows
    const uint32_t soff = static_cast<uint32_t>(s) * 64u;
#pragma unroll
    for (int mr = 0; mr < MR; ++mr) r.w[mr] = load16<kCached>(wr, w_voff[mr], soff);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) r.x[rb] = load16<kCached>(xr, x_voff[rb], soff);
  };
  floatx4_t acc[MR][RB];
#pragma unroll
  for (int mr = 0; mr < MR; ++mr)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[mr][rb] = floatx4_t{};
  auto compute_step = [&](const StepRegs<MR, RB>& r) {
    bf16x8_t a[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) a[rb] = to_fragment(r.x[rb]);
#pragma unroll
    for (int mr = 0; mr < MR; ++mr) {
      const bf16x8_t b = to_fragment(r.w[mr]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc[mr][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], b, acc[mr][rb], 0, 0, 0);
    }
  };

  StepRegs<MR, RB> slot[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    load_step(slot[j], s0 + j < s1 ? s0 + j : s1 - 1);
    __builtin_amdgcn_sched_barrier(0);  // one issue order for prologue and loop
  }
  // Whole rounds of D steps; a slot is refilled with the step D ahead right
  // after its compute (pinned there, so each step waits only for its own
  // loads), clamped to the last step of the slice past its end.
  const int rounds = (s1 - s0) / D;
  int s = s0;
  for (int r = 0; r < rounds; ++r, s += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      compute_step(slot[j]);
      load_step(slot[j], min(s + j + D, s1 - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int j = 0; j < D - 1; ++j)
    if (s + j < s1) compute_step(slot[j]);

  // Reduction over the WK waves in wave order, one row tile at a time.
  // Accumulator element e of (mr, rb) holds token n0 + 16 rb + 4 q + e,
  // feature m0 + tile_stride mr + c.  Every tile gives a lane the same j
  // values, so a SwiGLU lane keeps its gate sums in gsum for the up pass.
  constexpr int kJ = (RB * 4 + WK - 1) / WK;
  float gsum[kJ];
#pragma unroll
  for (int mr = 0; mr < MR; ++mr) {
    if (mr > 0) __syncthreads();  // the previous tile's sums are read
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int e = 0; e < 4; ++e) s_red[wave][rb * 4 + e][lane] = acc[mr][rb][e];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kJ; ++i) {
      const int j = wave + i * WK;
      if (j >= RB * 4) break;
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < WK; ++w) sum += s_red[w][j][lane];
      const int n = n0 + 16 * (j >> 2) + 4 * q + (j & 3);
      if constexpr (SWIGLU) {
        if (mr == 0) {
          gsum[i] = sum;
        } else if (n < N) {
          Y[static_cast<long long>(n) * M + m0 + c] =
              swiglu_one(bf2f(f2bf(gsum[i])), bf2f(f2bf(sum)));
        }
      } else if (n < N) {
        const long long o = static_cast<long long>(n) * M + m0 + 16 * mr + c;
        if constexpr (F32)
          static_cast<float*>(Yv)[o] = sum;
        else
          Y[o] = f2bf(sum);
      }
    }
  }
}

template <int WK, int MR, bool SWIGLU, bool F32>
void launch_dense_rb(int rb, dim3 grid, const uint16_t* W, const uint16_t* X, void* Y, int M,
                     int N, int K, int stride, hipStream_t stream) {
  const dim3 block(64 * WK);
  switch (rb) {
    case 1: hipLaunchKernelGGL((dense_gemm_kernel<WK, MR, 1, SWIGLU, F32>), grid, block, 0, stream, W, X, Y, M, N, K, stride); break;
    case 2: hipLaunchKernelGGL((dense_gemm_kernel<WK, MR, 2, SWIGLU, F32>), grid, block, 0, stream, W, X, Y, M, N, K, stride); break;
    case 3: hipLaunchKernelGGL((dense_gemm_kernel<WK, MR, 3, SWIGLU, F32>), grid, block, 0, stream, W, X, Y, M, N, K, stride); break;
    default: hipLaunchKernelGGL((dense_gemm_kernel<WK, MR, 4, SWIGLU, F32>), grid, block, 0, stream, W, X, Y, M, N, K, stride); break;
  }
}

template <int WK, bool SWIGLU, bool F32>
void launch_dense(int mr, int rb, dim3 grid, const uint16_t* W, const uint16_t* X, void* Y,
                  int M, int N, int K, int stride, hipStream_t stream) {
  if (SWIGLU || mr == 2)
    launch_dense_rb<WK, 2, SWIGLU, F32>(rb, grid, W, X, Y, M, N, K, stride, stream);
  else
    launch_dense_rb<WK, 1, false, F32>(rb, grid, W, X, Y, M, N, K, stride, stream);
}

// Row tiles per wave: two where M allows (each X fragment then feeds two
// MFMAs).  Token blocks per workgroup: up to four, halved once when the grid
// would leave CUs idle.  Filling the CUs is worth more than reading each W row
// once: the workgroups that share W rows sit at the same blockIdx.x, and since
// the row-tile count is a multiple of 8 on the shapes this serves (4096, 7168
// features) they land on the same XCD and find the rows in its L2 (Kimi
// gate/up, 64 tokens: 128 workgroups of 64 tokens 26.4 us, 256 of 32 tokens
// 20.4 us).
int pick_token_blocks(long long row_groups, int N, int cu) {
  int rb = N <= 16 ? 1 : N <= 32 ? 2 : N <= 48 ? 3 : 4;
  if (rb > 1 && row_groups * ceil_div(N, 16 * rb) < cu) rb = (rb + 1) / 2;
  return rb;
}

// Shared checks and launch.  rows = W rows read (M, or 2 I for SwiGLU),
// M = output features per token row of Y.
template <bool SWIGLU, bool F32 = false>
int dense_launch(const uint16_t* W, const uint16_t* X, void* Y, int rows, int M, int N, int K,
                 hipStream_t stream, const char* name) {
  if (!W || !X || !Y) return fail(kInvalidValue, "%s: null pointer", name);
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(kInvalidValue, "%s: bad shape M=%d N=%d K=%d", name, M, N, K);
  if (M % 16 != 0 || K % 32 != 0)
    return fail(kNotSupported, "%s: M %% 16 and K %% 32 must be 0 (M=%d K=%d)", name, M, K);
  if ((reinterpret_cast<uintptr_t>(W) & 15u) != 0 || (reinterpret_cast<uintptr_t>(X) & 15u) != 0)
    return fail(kNotSupported, "%s: W and X must be 16-byte aligned", name);
  // X is addressed through one 32-bit buffer range that must stay below the
  // out-of-range offset, and so is a workgroup's W span: its 16 MR rows, or
  // with SwiGLU its gate rows through its up rows (I + 16 rows).  The size of
  // W as a whole does not matter.
  const long long w_span = SWIGLU ? static_cast<long long>(M) + 16 : 32;
  if (static_cast<long long>(N) * K * 2 >= static_cast<long long>(kOutOfRange) ||
      w_span * K * 2 >= static_cast<long long>(kOutOfRange))
    return fail(kNotSupported, "%s: operand span over 2 GiB (rows=%d N=%d K=%d)", name, rows, N,
                K);
  const int cu = current_cu_count();
  if (cu <= 0) return fail(kInvalidValue, "%s: no device", name);
  const int mr = SWIGLU ? 2 : (M % 32 == 0 ? 2 : 1);
  const int gx = SWIGLU ? M / 16 : M / (16 * mr);
  const int rb = pick_token_blocks(gx, N, cu);
  const int ny = ceil_div(N, 16 * rb);
  if (ny > 65535) return fail(kNotSupported, "%s: too many token blocks (N=%d)", name, N);
  const dim3 grid(gx, ny);
  const int stride = SWIGLU ? M : 16;
  // Few workgroups: more waves each, splitting K (at least one step a wave).
  // Once the grid has a workgroup per CU, fewer and longer K shares (at least
  // 64 steps a wave) stream faster: Kimi's shared expert at 64 tokens, gate/up
  // 7168 x 4096 with SwiGLU (256 workgroups) 20.4 / 19.5 / 19.0 / 17.9 us at
  // 16 / 8 / 4 / 2 waves, down 2048 x 7168 (448 workgroups) 15.5 / 12.5 / 11.8 /
  // 11.5 us at 8 / 4 / 2 / 1 (graph replays over 4 weight copies, one box).
  const long long wgs = static_cast<long long>(grid.x) * grid.y;
  int wk = wgs <= cu ? 16 : (wgs <= 2LL * cu ? 8 : 4);
  if (wgs >= cu)
    while (wk > 1 && K / 32 < 64 * wk) wk >>= 1;
  while (wk > 1 && K / 32 < wk) wk >>= 1;
  switch (wk) {
    case 16: launch_dense<16, SWIGLU, F32>(mr, rb, grid, W, X, Y, M, N, K, stride, stream); break;
    case 8: launch_dense<8, SWIGLU, F32>(mr, rb, grid, W, X, Y, M, N, K, stride, stream); break;
    case 4: launch_dense<4, SWIGLU, F32>(mr, rb, grid, W, X, Y, M, N, K, stride, stream); break;
    case 2: launch_dense<2, SWIGLU, F32>(mr, rb, grid, W, X, Y, M, N, K, stride, stream); break;
    default: launch_dense<1, SWIGLU, F32>(mr, rb, grid, W, X, Y, M, N, K, stride, stream); break;
  }
  return launch_status(name);
}

// ---------------------------------------------------------------- prefill sizes
// From kLtMinTokens tokens up the GEMM is compute-bound and a plain library
// GEMM serves it: hipBLASLt's bf16 x bf16 -> bf16 kernel with fp32 accumulation
// (the reference runs cuBLAS there: cublasGemmEx with CUBLAS_COMPUTE_32F,
// linear.cu:321-344).  Column-major, as the reference states the call:
// C (M x N, ld M) = op_T(W: K x M, ld K) . op_N(X: K x N, ld K).  No workspace
// (an algorithm that needs none), so a call allocates nothing on the device; the
// library handle and each shape's descriptors and algorithm are made on the
// shape's first call on a device and reused.
constexpr int kLtMinTokens = 256;

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct LtDevice {
  std::mutex mu;
  hipblasLtHandle_t handle = nullptr;
  std::map<std::tuple<int, int, int>, LtPlan> plans;
};
LtDevice g_lt[64];

int lt_plan(int dev, int M, int N, int K, const char* name, LtDevice** out_d, LtPlan* out) {
  LtDevice& d = g_lt[dev];
  std::lock_guard<std::mutex> lock(d.mu);
  if (d.handle == nullptr && hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) {
    d.handle = nullptr;
    return fail(kLaunchFailed, "%s: hipblasLtCreate failed", name);
  }
  const auto key = std::make_tuple(M, N, K);
  auto it = d.plans.find(key);
  if (it == d.plans.end()) {
    LtPlan pl;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    bool ok = hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta,
                                              sizeof(ta)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb,
                                              sizeof(tb)) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&pl.a, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&pl.b, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&pl.c, HIP_R_16BF, M, N, M) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    if (ok) {
      const uint64_t ws = 0;
      ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                 &ws, sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulAlgoGetHeuristic(d.handle, pl.desc, pl.a, pl.b, pl.c, pl.c, pref, 1,
                                           res, &found) == HIPBLAS_STATUS_SUCCESS &&
           found > 0 && res[0].workspaceSize == 0;
    }
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (!ok) {
      if (pl.a) hipblasLtMatrixLayoutDestroy(pl.a);
      if (pl.b) hipblasLtMatrixLayoutDestroy(pl.b);
      if (pl.c) hipblasLtMatrixLayoutDestroy(pl.c);
      if (pl.desc) hipblasLtMatmulDescDestroy(pl.desc);
      return fail(kNotSupported, "%s: no hipBLASLt algorithm without workspace for M=%d N=%d K=%d",
                  name, M, N, K);
    }
    pl.algo = res[0].algo;
    it = d.plans.emplace(key, pl).first;
  }
  *out_d = &d;
  *out = it->second;
  return kSuccess;
}

int lt_gemm(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
            hipStream_t stream, const char* name) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(kInvalidValue, "%s: no current device", name);
  LtDevice* d = nullptr;
  LtPlan pl;
  const int rc = lt_plan(dev, M, N, K, name, &d, &pl);
  if (rc != kSuccess) return rc;
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st = hipblasLtMatmul(d->handle, pl.desc, &alpha, W, pl.a, X, pl.b, &beta,
                                             Y, pl.c, Y, pl.c, &pl.algo, nullptr, 0, stream);
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(kLaunchFailed, "%s: hipblasLtMatmul failed", name);
  return launch_status(name);
}

// gemm_cuda / gemm_graphsafe_cuda: the checks of dense_launch, then the token
// count picks the kernel.
int dense_gemm_bf16(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                    hipStream_t stream, const char* name) {
  if (N < kLtMinTokens || !W || !X || !Y || M <= 0 || N <= 0 || K <= 0 || M % 16 != 0 ||
      K % 32 != 0 || (reinterpret_cast<uintptr_t>(W) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(X) & 15u) != 0 ||
      static_cast<long long>(N) * K * 2 >= static_cast<long long>(kOutOfRange))
    return dense_launch<false>(W, X, Y, M, M, N, K, stream, name);
  return lt_gemm(W, X, Y, M, N, K, stream, name);
}

}  // namespace

// The router's logits GEMM (fp32 output); declared in common.h.
int dense_gemm_f32(const uint16_t* W, const uint16_t* X, float* Y, int M, int N, int K,
                   hipStream_t stream, const char* name) {
  return dense_launch<false, true>(W, X, Y, M, M, N, K, stream, name);
}

}  // namespace pega

using namespace pega;

// Reference: pegainfer-kernels/src/ffi/shared.rs:220-228 (gemm_cuda) and
// :230-238 (gemm_graphsafe_cuda); both compute the same GEMM.  Below 256
// tokens this library's weight-streaming kernel runs; from 256 up, hipBLASLt
// (no workspace).  Neither allocates device memory per call, so both are
// graph-safe once a shape has been called outside the capture (its first call
// on a device makes the hipBLASLt handle and plan).
PEGA_API int gemm_cuda(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                       hipStream_t stream) {
  return dense_gemm_bf16(W, X, Y, M, N, K, stream, "gemm_cuda");
}

PEGA_API int gemm_graphsafe_cuda(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N,
                                 int K, hipStream_t stream) {
  return dense_gemm_bf16(W, X, Y, M, N, K, stream, "gemm_graphsafe_cuda");
}

// No reference counterpart as one symbol: the shared expert's gate/up GEMM
// followed by the SwiGLU of its bf16 output.  The reference runs
// gemm_graphsafe_cuda, then silu_mul_fused_cuda (moe_nccl.rs:113-117 via
// silu_mul_hs_fused_into; csrc/shared/fused_proj.cu:11-31): per element
// bf16(f(bf16(g / (1 + e^-g))) * u) over the [N][2I] gate-then-up rows.  That
// is the same arithmetic as kimi_marlin_w13_swiglu_cuda
// (kimi_marlin_wna16.cu:345-361), which is what the epilogue here computes, so
// the result has the same bits as that pair.
PEGA_API int pega_dense_w13_swiglu(const uint16_t* W13, const uint16_t* X, uint16_t* act,
                                   int inter, int N, int K, hipStream_t stream) {
  if (inter > (1 << 29)) return fail(kInvalidValue, "pega_dense_w13_swiglu: bad inter=%d", inter);
  return dense_launch<true>(W13, X, act, 2 * inter, inter, N, K, stream, "pega_dense_w13_swiglu");
}
