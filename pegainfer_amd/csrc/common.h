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

// exp_exact_f32(x), bit for bit, at about half its cost.  For |x| <= 80 a
// degree-11 Taylor polynomial on r = x - n ln2 (|r| <= 0.347, ln2 split so that
// n * ln2_hi is exact) gives a = e^x within 2^-46.5 relative (truncation
// 0.347^12 / 12! / e^-0.347 = 2^-46.7, plus the Horner roundings).  The
// library's double exp is within one double ulp (2^-52) of e^x, so the two
// doubles differ by less than g = 2^-45 a.
// Both then round to the same float f = RN(a) unless a rounding midpoint of
// f's neighbourhood lies within g of a: that is checked exactly (a - f is exact
// in double), and only then, about once in 2^20 calls, does the double exp run.
// exp_exact_f32_try is that fast path alone, without branches: it returns f and
// sets *ok, which is false where the double exp must decide (|x| > 80, NaN, or a
// midpoint within g), so that callers can evaluate several exponentials side by
// side and take the rare fallbacks afterwards.
__device__ __forceinline__ float exp_exact_f32_try(float x, bool* ok) {
  const bool in = __builtin_fabsf(x) <= 80.0f;  // false for NaN too
  const double xd = in ? static_cast<double>(x) : 0.0;
  const double n = __builtin_rint(xd * 1.4426950408889634);
  double r = __builtin_fma(-n, 0x1.62e42fefa3800p-1, xd);  // ln2_hi: 43 bits, n * ln2_hi exact
  r = __builtin_fma(-n, 0x1.ef35793c76730p-45, r);          // ln2_lo
  double p = 1.0 / 39916800.0;                               // 1/11!
  p = __builtin_fma(p, r, 1.0 / 3628800.0);
  p = __builtin_fma(p, r, 1.0 / 362880.0);
  p = __builtin_fma(p, r, 1.0 / 40320.0);
  p = __builtin_fma(p, r, 1.0 / 5040.0);
  p = __builtin_fma(p, r, 1.0 / 720.0);
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const double a = __builtin_ldexp(p, static_cast<int>(n));
  const float f = static_cast<float>(a);
  const double d = a - static_cast<double>(f);  // exact: a and f within one float ulp
  const uint32_t fb = __builtin_bit_cast(uint32_t, f);
  // half the float ulp above f, and below it (a quarter when f is a power of two)
  const double half_up = __builtin_bit_cast(
      double, static_cast<uint64_t>(((fb >> 23) & 0xffu) + 1023u - 151u) << 52);
  const double half_dn = (fb & 0x7fffffu) ? half_up : 0.5 * half_up;
  const double g = a * 0x1p-45;
  *ok = in && d + g < half_up && d - g > -half_dn;
  return f;
}

__device__ __forceinline__ float exp_exact_f32_fast(float x) {
  bool ok;
  const float f = exp_exact_f32_try(x, &ok);
  return ok ? f : exp_exact_f32(x);
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
