// Load-time weight packaging: compressed-tensors INT4 checkpoint -> the
// on-device layout the grouped W4A16 GEMM consumes.
//
// The device layout is the reference's Marlin "uint4b8 no-act-order" layout,
// byte for byte (so packages built by either implementation are
// interchangeable and the reference's own known-answer tests apply):
//
//   weights  [E][K/16][2N] u32: 16(k) x 64(n) tiles of 128 words, tile
//            (kt, nt) at word (kt * N/64 + nt) * 128; word th*4 + w holds the
//            8 nibbles (n0 = nt*64 + w*16 + th/4, n1 = n0 + 8) x
//            (k = kt*16 + 2*(th%4) + {0, 1, 8, 9}) in nibble order
//            (n0,k0) (n0,k8) (n1,k0) (n1,k8) (n0,k1) (n0,k9) (n1,k1) (n1,k9).
//   scales   [E][K/32][N] bf16, every 64-column chunk permuted so that column
//            p of the chunk sits at 8*(p%8) + p/8.
//
// The GEMM kernels (wna16.hip) map MFMA 32x32x16 fragments directly onto
// these words, so no further conversion is needed on MI355X.
//
// Reference: pegainfer-kernels/csrc/kimi_k2/kimi_marlin_int4.cu:21-263;
// Rust ops src/ops/kimi_k2/experts.rs:850-1022.
#include "common.h"
#include "pega_moe.h"

namespace pega {
namespace {

// One thread per output word: gathers its 8 nibbles from 4 checkpoint words.
__global__ void reorder_weight_kernel(const uint32_t* __restrict__ ckpt,
                                      uint32_t* __restrict__ marlin, int size_k, int size_n,
                                      long long total_words) {
  const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total_words) return;
  const long long per_expert = static_cast<long long>(size_n) * (size_k / 8);
  const int e = static_cast<int>(idx / per_expert);
  const long long in_e = idx - e * per_expert;
  const int n_tiles = size_n / 64;
  const int word = static_cast<int>(in_e % 128);
  const long long tile = in_e / 128;
  const int nt = static_cast<int>(tile % n_tiles);
  const int kt = static_cast<int>(tile / n_tiles);
  const int th = word >> 2, w = word & 3;
  const int n0 = nt * 64 + w * 16 + (th >> 2);
  const int kb = kt * 16 + 2 * (th & 3);  // even, so kb and kb+1 share a word
  const int k_words = size_k / 8;
  const uint32_t* src = ckpt + e * per_expert;
  const uint32_t a0 = src[static_cast<long long>(n0) * k_words + (kb >> 3)];
  const uint32_t a1 = src[static_cast<long long>(n0) * k_words + ((kb + 8) >> 3)];
  const uint32_t b0 = src[static_cast<long long>(n0 + 8) * k_words + (kb >> 3)];
  const uint32_t b1 = src[static_cast<long long>(n0 + 8) * k_words + ((kb + 8) >> 3)];
  const int sh = (kb & 7) * 4;
  const uint32_t nk0 = (a0 >> sh) & 0xf, nk1 = (a0 >> (sh + 4)) & 0xf;
  const uint32_t nk8 = (a1 >> sh) & 0xf, nk9 = (a1 >> (sh + 4)) & 0xf;
  const uint32_t mk0 = (b0 >> sh) & 0xf, mk1 = (b0 >> (sh + 4)) & 0xf;
  const uint32_t mk8 = (b1 >> sh) & 0xf, mk9 = (b1 >> (sh + 4)) & 0xf;
  marlin[idx] = nk0 | (nk8 << 4) | (mk0 << 8) | (mk8 << 12) | (nk1 << 16) | (nk9 << 20) |
                (mk1 << 24) | (mk9 << 28);
}

__global__ void reorder_scale_kernel(const uint16_t* __restrict__ ckpt,
                                     uint16_t* __restrict__ marlin, int size_n, int scale_k,
                                     long long total) {
  const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const long long per_expert = static_cast<long long>(size_n) * scale_k;
  const long long e = idx / per_expert;
  const long long in_e = idx - e * per_expert;
  const int o = static_cast<int>(in_e & 63);
  const long long src_flat = (in_e & ~63LL) + (o >> 3) + 8 * (o & 7);
  const int g = static_cast<int>(src_flat / size_n);
  const int row = static_cast<int>(src_flat - static_cast<long long>(g) * size_n);
  marlin[idx] = ckpt[e * per_expert + static_cast<long long>(row) * scale_k + g];
}

// Row concatenation [rows][2][cols]: gate half then up half, 16-byte copies.
__global__ void concat_rows_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b,
                                   uint4* __restrict__ out, long long rows, int cols16) {
  const long long total = rows * cols16;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long r = idx / cols16;
    const int c = static_cast<int>(idx - r * cols16);
    out[r * 2 * cols16 + c] = a[idx];
    out[r * 2 * cols16 + cols16 + c] = b[idx];
  }
}

__global__ void concat_rows_u16_kernel(const uint16_t* __restrict__ a,
                                       const uint16_t* __restrict__ b,
                                       uint16_t* __restrict__ out, long long rows, int cols) {
  const long long total = rows * cols;
  for (long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
       idx < total; idx += static_cast<long long>(gridDim.x) * blockDim.x) {
    const long long r = idx / cols;
    const int c = static_cast<int>(idx - r * cols);
    out[r * 2 * cols + c] = a[idx];
    out[r * 2 * cols + cols + c] = b[idx];
  }
}

bool common_shape_ok(int in_dim, int out_dim, int local_experts, int group_size) {
  return in_dim > 0 && out_dim > 0 && local_experts > 0 && group_size == 32 &&
         in_dim % 16 == 0 && out_dim % 64 == 0 && in_dim % group_size == 0;
}

unsigned grid_for(long long n, int threads) {
  long long g = (n + threads - 1) / threads;
  return static_cast<unsigned>(g < 1 ? 1 : (g > 0x7fffffffLL ? 0x7fffffffLL : g));
}

}  // namespace

int reorder_weight(const uint8_t* ckpt, uint8_t* marlin, int in_dim, int out_dim,
                   int local_experts, int group_size, hipStream_t stream) {
  if (!ckpt || !marlin) return fail(kInvalidValue, "reorder_weight: null pointer");
  if (!common_shape_ok(in_dim, out_dim, local_experts, group_size))
    return fail(kInvalidValue, "reorder_weight: bad shape in=%d out=%d E=%d group=%d", in_dim,
                out_dim, local_experts, group_size);
  const long long total = static_cast<long long>(local_experts) * out_dim * (in_dim / 8);
  hipLaunchKernelGGL(reorder_weight_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                     reinterpret_cast<const uint32_t*>(ckpt), reinterpret_cast<uint32_t*>(marlin),
                     in_dim, out_dim, total);
  return launch_status("reorder_weight");
}

int reorder_scale(const uint16_t* ckpt, uint16_t* marlin, int in_dim, int out_dim,
                  int local_experts, int group_size, hipStream_t stream) {
  if (!ckpt || !marlin) return fail(kInvalidValue, "reorder_scale: null pointer");
  if (in_dim <= 0 || out_dim <= 0 || local_experts <= 0 || group_size != 32 ||
      in_dim % group_size != 0)
    return fail(kInvalidValue, "reorder_scale: bad shape");
  const int scale_k = in_dim / group_size;
  const long long per_expert = static_cast<long long>(out_dim) * scale_k;
  if (per_expert % 64 != 0)
    return fail(kInvalidValue, "reorder_scale: out*groups (%lld) not a multiple of 64",
                per_expert);
  const long long total = per_expert * local_experts;
  hipLaunchKernelGGL(reorder_scale_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                     ckpt, marlin, out_dim, scale_k, total);
  return launch_status("reorder_scale");
}

int fuse_w13(const uint8_t* gate_w, const uint8_t* up_w, uint8_t* w13_w, const uint16_t* gate_s,
             const uint16_t* up_s, uint16_t* w13_s, int in_dim, int inter, int local_experts,
             int group_size, hipStream_t stream) {
  if (!gate_w || !up_w || !w13_w || !gate_s || !up_s || !w13_s)
    return fail(kInvalidValue, "fuse_w13: null pointer");
  if (!common_shape_ok(in_dim, inter, local_experts, group_size))
    return fail(kInvalidValue, "fuse_w13: bad shape in=%d inter=%d E=%d", in_dim, inter,
                local_experts);
  // Weights: rows = E * K/16, each gate row is 2*inter u32 = inter/2 uint4.
  const long long wrows = static_cast<long long>(local_experts) * (in_dim / 16);
  const int wcols16 = inter / 2;
  hipLaunchKernelGGL(concat_rows_kernel, dim3(grid_for(wrows * wcols16, 256)), dim3(256), 0,
                     stream, reinterpret_cast<const uint4*>(gate_w),
                     reinterpret_cast<const uint4*>(up_w), reinterpret_cast<uint4*>(w13_w),
                     wrows, wcols16);
  int st = launch_status("fuse_w13 weights");
  if (st != kSuccess) return st;
  const long long srows = static_cast<long long>(local_experts) * (in_dim / group_size);
  hipLaunchKernelGGL(concat_rows_u16_kernel, dim3(grid_for(srows * inter, 256)), dim3(256), 0,
                     stream, gate_s, up_s, w13_s, srows, inter);
  return launch_status("fuse_w13 scales");
}

}  // namespace pega

// ---------------------------------------------------------------- C ABI
// Reference declarations: pegainfer-kernels/src/ffi/kimi.rs:68-101; guards
// kimi_marlin_int4.cu:15-19,179-184,201-213,235-242 (local_experts == 48).  The
// reference maps every failure of these calls, a launch failure included, to
// CUDA_ERROR_INVALID_VALUE (kimi_marlin_int4.cu:190,220,254,262), and so do these.
namespace {
int as_invalid_value(int rc) { return rc == pega::kSuccess ? rc : pega::kInvalidValue; }
}  // namespace

PEGA_API int kimi_marlin_int4_reorder_weight_cuda(const uint8_t* weight_packed_checkpoint,
                                                  uint8_t* weight_packed_marlin, int in_dim,
                                                  int out_dim, int local_experts,
                                                  int group_size, hipStream_t stream) {
  if (local_experts != 48)
    return pega::fail(pega::kInvalidValue, "kimi reorder_weight: local_experts must be 48");
  return as_invalid_value(pega::reorder_weight(weight_packed_checkpoint, weight_packed_marlin,
                                               in_dim, out_dim, local_experts, group_size,
                                               stream));
}

PEGA_API int kimi_marlin_int4_reorder_scale_cuda(const uint16_t* weight_scale_checkpoint,
                                                 uint16_t* weight_scale_marlin, int in_dim,
                                                 int out_dim, int local_experts, int group_size,
                                                 hipStream_t stream) {
  if (local_experts != 48)
    return pega::fail(pega::kInvalidValue, "kimi reorder_scale: local_experts must be 48");
  return as_invalid_value(pega::reorder_scale(weight_scale_checkpoint, weight_scale_marlin,
                                              in_dim, out_dim, local_experts, group_size,
                                              stream));
}

PEGA_API int kimi_marlin_int4_fuse_w13_cuda(const uint8_t* gate_weight_packed_marlin,
                                            const uint8_t* up_weight_packed_marlin,
                                            uint8_t* w13_weight_packed_marlin,
                                            const uint16_t* gate_scale_marlin,
                                            const uint16_t* up_scale_marlin,
                                            uint16_t* w13_scale_marlin, int in_dim,
                                            int intermediate_dim, int local_experts,
                                            int group_size, hipStream_t stream) {
  if (local_experts != 48)
    return pega::fail(pega::kInvalidValue, "kimi fuse_w13: local_experts must be 48");
  return as_invalid_value(pega::fuse_w13(gate_weight_packed_marlin, up_weight_packed_marlin,
                                         w13_weight_packed_marlin, gate_scale_marlin,
                                         up_scale_marlin, w13_scale_marlin, in_dim,
                                         intermediate_dim, local_experts, group_size, stream));
}

// Shape-general variants (any expert count; no reference counterpart).
PEGA_API int pega_marlin_int4_reorder_weight(const uint8_t* ckpt, uint8_t* marlin, int in_dim,
                                             int out_dim, int local_experts, int group_size,
                                             hipStream_t stream) {
  return pega::reorder_weight(ckpt, marlin, in_dim, out_dim, local_experts, group_size, stream);
}

PEGA_API int pega_marlin_int4_reorder_scale(const uint16_t* ckpt, uint16_t* marlin, int in_dim,
                                            int out_dim, int local_experts, int group_size,
                                            hipStream_t stream) {
  return pega::reorder_scale(ckpt, marlin, in_dim, out_dim, local_experts, group_size, stream);
}

PEGA_API int pega_marlin_int4_fuse_w13(const uint8_t* gate_w, const uint8_t* up_w,
                                       uint8_t* w13_w, const uint16_t* gate_s,
                                       const uint16_t* up_s, uint16_t* w13_s, int in_dim,
                                       int intermediate_dim, int local_experts, int group_size,
                                       hipStream_t stream) {
  return pega::fuse_w13(gate_w, up_w, w13_w, gate_s, up_s, w13_s, in_dim, intermediate_dim,
                        local_experts, group_size, stream);
}
