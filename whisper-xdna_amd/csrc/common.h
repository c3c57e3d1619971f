// Shared device helpers for the gfx950 kernels: bf16 bit conversions, vector
// types for the MFMA builtins, and wave-level reductions.
//
// bf16 values are carried as their uint16_t bit pattern in memory. Rounding
// fp32 -> bf16 uses v_cvt_pk_bf16_f32 (round to nearest even) through the
// __bf16 conversion, or a plain shift for truncation toward zero.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// Two fp32 -> packed bf16 pair in one v_cvt_pk_bf16_f32 (low half = a).
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  f32x2 v = {a, b};
  bf16x2 h = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint16_t f2bf_trunc(float f) {
  return static_cast<uint16_t>(__float_as_uint(f) >> 16);
}

// Round to bf16 and back: the value as the next consumer of a bf16 sees it.
__device__ __forceinline__ float rb_rne(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ float rb_trunc(float f) {
  return __uint_as_float(__float_as_uint(f) & 0xFFFF0000u);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Exact erf-GELU in fp32: 0.5*x*erfc(-x/sqrt2). The erfc form keeps full
// relative precision in the negative tail, where 1 + erf(x/sqrt2) cancels.
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * erfcf(-x * 0.70710678118654752440f);
}

// erf-GELU for GEMM epilogues, where its VALU cost competes with the MFMAs:
// GELU(x) = x * Phi(x), Phi(-|x|) = 0.5 * erfc(|x| / sqrt2), with erfc from
// the Chebyshev fit of Numerical Recipes (2nd ed., sec. 6.2, "erfcc":
// erfc(z) = t * exp(-z^2 + P(t)), t = 1 / (1 + z/2), fractional error
// < 1.2e-7 for all z >= 0). One reciprocal, one exp2 (P pre-scaled by
// log2 e), ten FMAs. Within 1 bf16 ulp of the exact GELU for |x| < 13 (fp32
// evaluation, relative error < 3e-5); beyond that the result is below 1e-36.
__device__ __forceinline__ float gelu_erf_fast(float x) {
  constexpr float kL2e = 1.4426950408889634f;
  const float z = fabsf(x) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f * kL2e;
  p = fmaf(p, t, -0.82215223f * kL2e);
  p = fmaf(p, t, 1.48851587f * kL2e);
  p = fmaf(p, t, -1.13520398f * kL2e);
  p = fmaf(p, t, 0.27886807f * kL2e);
  p = fmaf(p, t, -0.18628806f * kL2e);
  p = fmaf(p, t, 0.09678418f * kL2e);
  p = fmaf(p, t, 0.37409196f * kL2e);
  p = fmaf(p, t, 1.00002368f * kL2e);
  p = fmaf(p, t, -1.26551223f * kL2e);
  const float e = 0.5f * t * __builtin_amdgcn_exp2f(fmaf(-z * z, kL2e, p));  // Phi(-|x|)
  return x * (x >= 0.f ? 1.0f - e : e);
}

}  // namespace wx
