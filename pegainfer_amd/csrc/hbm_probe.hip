// Measurement only, not part of the expert path: a plain streaming read, the
// attainable HBM read rate that bench.py reports beside the GEMM kernels'
// roofline fractions.  Workgroup b reads its contiguous chunk of the buffer
// with 16-byte non-temporal loads, four per thread in flight, and folds the
// words into one XOR per thread so the loads cannot be dropped.  Built into
// its own library (libpega_hbm_probe.so); the expert-path library does not
// contain it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4_t* __restrict__ src,
                                                       size_t n16, uint32_t* __restrict__ out) {
  const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = static_cast<size_t>(blockIdx.x) * chunk;
  const size_t b1 = b0 + chunk < n16 ? b0 + chunk : n16;
  uint32_t acc = 0;
  size_t i = b0 + threadIdx.x;
  for (; i + 3 * 256 < b1; i += 4 * 256) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < b1; i += 256) {
    const u32x4_t a = src[i];
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  out[static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x] = acc;
}

}  // namespace

// src: `bytes` bytes (a multiple of 16, 16-byte aligned); out: grid * 256 words.
extern "C" __attribute__((visibility("default"))) int pega_hbm_read_probe(
    const void* src, unsigned long long bytes, void* out, int grid, hipStream_t stream) {
  if (!src || !out || grid <= 0 || (bytes & 15ull) != 0 ||
      (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
    return 1;
  hipLaunchKernelGGL(hbm_read_kernel, dim3(grid), dim3(256), 0, stream,
                     static_cast<const u32x4_t*>(src), static_cast<size_t>(bytes / 16),
                     static_cast<uint32_t*>(out));
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
