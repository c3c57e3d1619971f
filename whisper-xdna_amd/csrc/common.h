// Shared device helpers for the gfx950 kernels: bf16 bit conversions, vector
// types for the MFMA builtins, and wave-level reductions.
//
// bf16 values are carried as their uint16_t bit pattern in memory. Rounding
// fp32 -> bf16 uses v_cvt_pk_bf16_f32 (round to nearest even) through the
// __bf16 conversion, or a plain shift for truncation toward zero.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

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
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

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

// Full-wave reductions, result wave-uniform. Four in-row DPP steps (quad
// swaps of 1 and 2 lanes, half-row mirror, row mirror) leave every lane of a
// 16-lane row with the row's value; the four rows' values are read with
// v_readlane and combined in scalar order. No LDS round trip on the path.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppRowMirror = 0x140;  // row_mirror

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppQuadSwap1>(v);
  v += dpp_f<kDppQuadSwap2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Workgroups are dispatched to the 8 XCDs round-robin by linear id, and each
// XCD has its own L2. xcd_remap(id, total) renumbers ids so that the ids one
// XCD receives (id % 8 == x) are one contiguous run of [0, total): work
// items that are numbered next to each other (tiles sharing operands, query
// blocks of one head) then share an L2.
constexpr int kXcds = 8;

// Workgroup barrier for the DMA-ring loops (GEMM, attention), whose LDS
// traffic is direct-to-LDS loads, which each wave has already waited for as
// far as it needs with an explicit vmcnt, and ds_reads: the wave's reads are
// waited for here (lgkmcnt(0): no wave may refill a slot another is still
// reading), then s_barrier, as one asm statement with a memory clobber so
// the compiler moves no memory access across it. __syncthreads() adds a
// workgroup-scope fence, for which the compiler first waits for every
// outstanding LDS DMA of the wave: in a prologue that drains the whole ring,
// so the first step would wait for the last prologue stage to land.
__device__ __forceinline__ void dma_ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int per = (total + kXcds - 1) / kXcds;
  int tall = total % kXcds;
  if (tall == 0) tall = kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  return xcd < tall ? xcd * per + local
                    : tall * per + (xcd - tall) * (per - 1) + local;
}


// The int8 quantisers' x / s (then rint), equal to the correctly rounded
// fp32 quotient. With r = 1 / s correctly rounded (one division per row),
// q0 = RN(x r) is within an ulp of x / s, the residual x - q0 s is exact as
// an FMA, and RN(q0 + (x - q0 s) r) is the correctly rounded quotient
// (Markstein's theorem), as long as nothing over- or underflows: s within
// [2^-100, 2^100] (`fast`, per row); outside it, the division itself.
// Checked against the exact quotient (rational arithmetic) over 4e5 cases,
// ties to half-integers and scales from 2^-100 to 2^125 included.
struct QuantScale {
  float s, r;
  bool fast;
};
__device__ __forceinline__ QuantScale quant_scale(float s) {
  return {s, 1.0f / s, s >= 0x1p-100f && s <= 0x1p100f};
}
__device__ __forceinline__ float quant_quotient(float x, const QuantScale& q) {
#pragma clang fp contract(off)
  if (!q.fast) return x / q.s;
  const float q0 = x * q.r;
  return fmaf(fmaf(-q0, q.s, x), q.r, q0);
}

// Compile-time loop: f(std::integral_constant<int, i>) for i in [0, N). Keeps
// every accumulator index a constant whatever the unroller decides, so the
// accumulators never get dynamically indexed (which would spill them).
template <class F, int... Is>
__device__ __forceinline__ void sfor_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  sfor_impl(f, std::make_integer_sequence<int, N>{});
}

// erf-GELU, GELU(x) = x Phi(x), for every kernel that applies it (row
// kernel and GEMM epilogues). With z = |x| / sqrt2 and t = 1 / (1 + z/2):
//   q = x Phi(-|x|) = x (erfc(z) / 2) = x t 2^(P(t) - z^2 log2 e - 1)
//   GELU(x) = max(x, 0) - |q|          (x - q for x >= 0, q for x < 0)
// P is this project's own least-squares fit (weighted towards minimax) of
// log2(erfc(z) e^(z^2) / t) on z in [0, 9.8], degree 3: |dP| < 3.9e-4, so q
// has relative error < 2.8e-4, far below a bf16 ulp (2^-8 relative); fp32
// evaluation over 4M inputs (the tail included) is within 1 bf16 ulp of
// the exact GELU. The exponent is taken as 2^(arg + 32) and the 2^-33 is
// applied by the final FMA, so results in fp32's denormal range come out of
// an IEEE operation instead of an exp2 that may flush them. In terms of x:
// t = 1 / (1 + |x| / (2 sqrt2)) and z^2 log2 e = x^2 (log2 e / 2). For
// |x| >= 14 the exp2 underflows to 0 and the result is relu(x) exactly; x
// enters the product clamped to [-16, 16], so +-inf (t = 0) map to relu
// too. One reciprocal, one exp2 and 11 other VALU operations.
__device__ __forceinline__ float gelu_erf(float x) {
  constexpr float kHalfL2e = 0.72134752044448170f;  // log2(e) / 2
  const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), 0.35355339059327376f, 1.0f));
  float p = -0.5002267360687256f;
  p = fmaf(p, t, 0.9977306127548218f);
  p = fmaf(p, t, 1.31719970703125f);
  p = fmaf(p, t, -1.8143213987350464f + 32.0f);
  const float e = __builtin_amdgcn_exp2f(fmaf(x * x, -kHalfL2e, p));
  const float w = __builtin_amdgcn_fmed3f(x, -16.0f, 16.0f) * t * e;  // q 2^33
  return fmaf(-fabsf(w), 1.1641532182693481e-10f, fmaxf(x, 0.f));  // 2^-33
}

// poly4 GELU constants: kernels/gelu_poly4_coeffs.h:4-13 (all bf16-exact;
// the breaks {1, 2, 4} and scales {2, 2, 1} appear inline below).
constexpr float kP4Shift[3] = {0.5f, 1.5f, 3.0f};
constexpr float kP4Coef[3][5] = {
    {-0.0020446777f, -0.013000488f, 0.077148438f, -0.06640625f, -0.15429688f},
    {0.0021514893f, -0.0071716309f, -0.0040283203f, 0.063964844f, -0.10009766f},
    {-0.0029296875f, 0.010681152f, -0.015869141f, 0.012023926f, -0.0040283203f},
};

// GELU(x) = relu(x) + q(|x|) with q the 3-piece degree-4 bump, rounded to
// bf16 at exactly the points gelu_poly4_eval.inc rounds. x must already be
// bf16-exact. poly4_q(s) is the bump for s = |x|; poly4_gelu_pre returns the
// fp32 sum before the final rounding.
// gelu_poly4_eval.inc evaluates the pieces p = 2, 1, 0 in turn and keeps the
// last one whose break exceeds s; that is the smallest p with s < break[p]
// (none for s >= 4 or NaN: q = 0). Only that piece is evaluated here, with
// its constants picked by two compares; the arithmetic on it is unchanged,
// so the result is bit-identical.
template <bool RNE>
__device__ __forceinline__ float poly4_q(float s) {
  const bool in0 = s < 1.0f, in1 = s < 2.0f, in2 = s < 4.0f;
  // piece p's constant: kP4Coef[p][k] etc., selected without indexing (an
  // indexed constant array would be read from memory per element)
  auto sel = [&](float c0, float c1, float c2) { return in0 ? c0 : (in1 ? c1 : c2); };
  float t = s - sel(kP4Shift[0], kP4Shift[1], kP4Shift[2]);
  t = RNE ? rb_rne(t) : rb_trunc(t);
  float u = t * (in1 ? 2.0f : 1.0f);  // kP4Scale = {2, 2, 1}
  u = RNE ? rb_rne(u) : rb_trunc(u);
  float acc = sel(kP4Coef[0][0], kP4Coef[1][0], kP4Coef[2][0]);
#pragma unroll
  for (int k = 1; k <= 4; ++k) {
    const float ah = RNE ? rb_rne(acc) : rb_trunc(acc);
    // ah * u is exact in fp32 (two bf16 factors), so one rounding
    acc = fmaf(ah, u, sel(kP4Coef[0][k], kP4Coef[1][k], kP4Coef[2][k]));
  }
  return in2 ? (RNE ? rb_rne(acc) : rb_trunc(acc)) : 0.f;
}

template <bool RNE>
__device__ __forceinline__ float poly4_gelu_pre(float x) {
  return fmaxf(x, 0.f) + poly4_q<RNE>(fabsf(x));
}

}  // namespace wx
