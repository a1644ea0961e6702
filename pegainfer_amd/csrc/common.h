// Shared definitions of the MI355X (gfx950) quantized-MoE expert-path library.
//
// ABI conventions (mirroring pegainfer-kernels/src/ffi/kimi.rs and src/ffi.rs:5):
//   * bf16 tensors cross the boundary as uint16_t bit patterns;
//   * every entry point returns an int with CUresult-compatible values;
//   * entry points never allocate, never synchronise and never throw; the
//     reason for a non-zero return is kept in a thread-local string that
//     pegainfer_kernels_last_error() returns (csrc/shared/ffi_last_error.cu:13
//     in the reference).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PEGA_API extern "C" __attribute__((visibility("default")))

namespace pega {

// CUresult-compatible status codes (cudarc::driver::sys::CUresult values).
enum Status : int {
  kSuccess = 0,
  kInvalidValue = 1,
  kNotInitialized = 3,
  kNotSupported = 801,
  kLaunchFailed = 719,
};

// Records the reason for a failure (printf-style) and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps the launch status of the kernel just enqueued to a Status.
int launch_status(const char* what);

// Number of compute units of the current device (cached per device).
int current_cu_count();

// Y[n][m] = sum_k f(W[m][k]) * f(X[n][k]) in fp32, unrounded: W [M][K], X [N][K] bf16,
// Y [N][M] fp32 (dense.hip; the router's logits GEMM).  Returns a Status.
int dense_gemm_f32(const uint16_t* W, const uint16_t* X, float* Y, int M, int N, int K,
                   hipStream_t stream, const char* name);

// ---------------------------------------------------------------- bf16 helpers
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two fp32 -> packed bf16 pair (lo = a, hi = b), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  bf16x2_t v;
  v[0] = static_cast<__bf16>(a);
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf_lo(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) {
  return __builtin_bit_cast(float, p & 0xffff0000u);
}

// e^x as the correctly rounded float of a double-precision exp.  Used where
// the reference calls expf and the result decides an index (router scores);
// the CPU checker uses the same definition.
__device__ __forceinline__ float exp_exact_f32(float x) {
  return static_cast<float>(::exp(static_cast<double>(x)));
}

// SwiGLU of one column pair: bf16( f(bf16(g / (1 + e^-g))) * u ), g = gate,
// u = up (pegainfer-kernels/csrc/kimi_k2/kimi_marlin_wna16.cu:345-361), with
// e^-g the exp_exact_f32 value (the CPU checker's definition).
//
// Only bf16(silu) reaches the result, so most gates skip the double-precision
// exponential.  For 2^-60 <= |g| <= 64 the hardware base-2 exponential gives a
// silu within (2|g| + 9) ulp of the exact one: -g * log2(e) is rounded twice
// (|g| * 2^-23 relative error in e^-g), v_exp_f32 adds at most 2 ulp, the
// exact e^-g is within half an ulp, and 1 + e and the quotient are rounded once
// in each computation.  Two floats that close round to the same bf16 unless a
// rounding midpoint (low half 0x8000) lies between them, so when the fast
// silu's low half is farther than 2|g| + 16 ulp from 0x8000 its bf16 is the
// exact one's; otherwise (about 1 gate in 2000 at |g| ~ 1), and outside that
// range of |g|, the exact exponential decides.  The kernels only pass bf16
// gates, and tests/test_gpu_elementwise.py checks all 65536 of them.
__device__ __forceinline__ uint16_t swiglu_one(float g, float u) {
  const float ag = __builtin_fabsf(g);
  bool exact = !(ag >= 0x1p-60f && ag <= 64.0f);  // NaN too
  float silu = 0.0f;
  if (!exact) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896340736f);
    silu = g / (1.0f + e);
    const int low = static_cast<int>(__builtin_bit_cast(uint32_t, silu) & 0xffffu);
    const int room = 2 * static_cast<int>(ag) + 16;
    exact = low > 0x8000 - room && low < 0x8000 + room;
  }
  if (exact) {
    const float e = (g == 0.0f) ? 1.0f : exp_exact_f32(-g);
    silu = g / (1.0f + e);
  }
  return f2bf(bf2f(f2bf(silu)) * u);
}

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace pega
