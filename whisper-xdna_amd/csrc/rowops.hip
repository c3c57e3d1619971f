// Row kernels for gfx950: LayerNorm, GELU (erf and the poly4 variants), row
// softmax, fp32 -> bf16 conversion, and the mel re-layout for the conv front
// end.
//
// Reference semantics (file:line in drakosha/whisper-xdna):
//   LayerNorm  src/npu_whisper_encoder.py:278-281, with the affine that
//              kernels/layer_norm_gb.cc:48-86 leaves to the next GEMM
//   erf-GELU   src/npu_whisper_encoder.py:284-287 (exact erf formulation)
//   poly4 GELU kernels/gelu_poly4_eval.inc:27-65, coefficients
//              kernels/gelu_poly4_coeffs.h:4-13; g4f input rounding
//              kernels/gelu_row4f.cc:58-84, g4r RNE kernels/gelu_row4_rne.cc,
//              g4 truncation kernels/gelu_row4.cc
//   softmax    src/npu_whisper_encoder.py:416-419, `valid` window of
//              src/rowops.py:60-73
//
// All of these are HBM-bound: one read and one write of each element. The
// row kernels put one wave on one row and keep the row in registers, so the
// reductions are wave shuffles and each element is read once.
#include "common.h"
#include "kernels.h"

namespace wx {

// ======================================================== LayerNorm
// One wave per row; lane l owns 8-element chunks l, l+64, ... of the row.
template <int MAXCH, bool XF32, bool YF32, bool RESID>
__global__ __launch_bounds__(256) void ln_kernel(
    const void* __restrict__ xp, int64_t ldx, const float* __restrict__ rp,
    int64_t ldr, float* __restrict__ sp, int64_t lds,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    void* __restrict__ yp, int64_t ldy, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols >> 3;
  float v[MAXCH][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int ch = lane + c * 64;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = 0.f;
    if (ch < nch) {
      const int64_t col = (int64_t)ch * 8;
      if (XF32) {
        const float* x = static_cast<const float*>(xp) + row * ldx + col;
        f32x4 a = *reinterpret_cast<const f32x4*>(x);
        f32x4 b = *reinterpret_cast<const f32x4*>(x + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[c][j] = a[j]; v[c][j + 4] = b[j]; }
      } else {
        const uint16_t* x = static_cast<const uint16_t*>(xp) + row * ldx + col;
        u16x8 a = *reinterpret_cast<const u16x8*>(x);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[c][j] = bf2f(a[j]);
      }
      if (RESID) {
        const float* r = rp + row * ldr + col;
        f32x4 a = *reinterpret_cast<const f32x4*>(r);
        f32x4 b = *reinterpret_cast<const f32x4*>(r + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[c][j] += a[j]; v[c][j + 4] += b[j]; }
        if (sp) {
          float* o = sp + row * lds + col;
          f32x4 lo = {v[c][0], v[c][1], v[c][2], v[c][3]};
          f32x4 hi = {v[c][4], v[c][5], v[c][6], v[c][7]};
          *reinterpret_cast<f32x4*>(o) = lo;
          *reinterpret_cast<f32x4*>(o + 4) = hi;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += v[c][j];
    }
  }
  const float inv_n = 1.0f / (float)cols;
  const float mean = wave_sum(sum) * inv_n;
  // second pass over the registers: exact two-pass variance
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    if (lane + c * 64 < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float dlt = v[c][j] - mean;
        sq += dlt * dlt;
      }
    }
  }
  const float var = wave_sum(sq) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= nch) continue;
    const int64_t col = (int64_t)ch * 8;
    float o[8];
    f32x4 g0 = {1.f, 1.f, 1.f, 1.f}, g1 = g0, b0 = {0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (gamma) {
      g0 = *reinterpret_cast<const f32x4*>(gamma + col);
      g1 = *reinterpret_cast<const f32x4*>(gamma + col + 4);
    }
    if (beta) {
      b0 = *reinterpret_cast<const f32x4*>(beta + col);
      b1 = *reinterpret_cast<const f32x4*>(beta + col + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[j] = (v[c][j] - mean) * rstd * g0[j] + b0[j];
      o[j + 4] = (v[c][j + 4] - mean) * rstd * g1[j] + b1[j];
    }
    if (YF32) {
      float* y = static_cast<float*>(yp) + row * ldy + col;
      f32x4 lo = {o[0], o[1], o[2], o[3]};
      f32x4 hi = {o[4], o[5], o[6], o[7]};
      *reinterpret_cast<f32x4*>(y) = lo;
      *reinterpret_cast<f32x4*>(y + 4) = hi;
    } else {
      uint16_t* y = static_cast<uint16_t*>(yp) + row * ldy + col;
      u32x4 pk = {f2bf2(o[0], o[1]), f2bf2(o[2], o[3]), f2bf2(o[4], o[5]),
                  f2bf2(o[6], o[7])};
      *reinterpret_cast<u32x4*>(y) = pk;
    }
  }
}

template <int MAXCH>
static hipError_t ln_dispatch(const void* x, int x_dtype, int64_t ldx,
                              const float* resid, int64_t ldr, float* sum_out,
                              int64_t lds, const float* gamma,
                              const float* beta, float eps, void* y,
                              int y_dtype, int64_t ldy, int rows, int cols,
                              hipStream_t s) {
  dim3 grid((rows + 3) / 4), block(256);
  const bool xf = x_dtype == DT_F32, yf = y_dtype == DT_F32, r = resid != nullptr;
#define WX_LN(XF, YF, R)                                                      \
  if (xf == XF && yf == YF && r == R) {                                       \
    ln_kernel<MAXCH, XF, YF, R><<<grid, block, 0, s>>>(                       \
        x, ldx, resid, ldr, sum_out, lds, gamma, beta, eps, y, ldy, rows, cols); \
    return hipGetLastError();                                                 \
  }
  WX_LN(false, false, false) WX_LN(false, true, false)
  WX_LN(true, false, false) WX_LN(true, true, false)
  WX_LN(false, false, true) WX_LN(false, true, true)
  WX_LN(true, false, true) WX_LN(true, true, true)
#undef WX_LN
  return hipErrorInvalidValue;
}

hipError_t launch_layernorm(const void* x, int x_dtype, int64_t ldx,
                            const float* resid, int64_t ldr, float* sum_out,
                            int64_t lds, const float* gamma, const float* beta,
                            float eps, void* y, int y_dtype, int64_t ldy,
                            int rows, int cols, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (cols <= 1024)
    return ln_dispatch<2>(x, x_dtype, ldx, resid, ldr, sum_out, lds, gamma,
                          beta, eps, y, y_dtype, ldy, rows, cols, s);
  if (cols <= 2048)
    return ln_dispatch<4>(x, x_dtype, ldx, resid, ldr, sum_out, lds, gamma,
                          beta, eps, y, y_dtype, ldy, rows, cols, s);
  return ln_dispatch<8>(x, x_dtype, ldx, resid, ldr, sum_out, lds, gamma, beta,
                        eps, y, y_dtype, ldy, rows, cols, s);
}

// ======================================================== GELU
// poly4 constants: kernels/gelu_poly4_coeffs.h:4-13 (all bf16-exact).
__constant__ float kP4Break[3] = {1.0f, 2.0f, 4.0f};
__constant__ float kP4Shift[3] = {0.5f, 1.5f, 3.0f};
__constant__ float kP4Scale[3] = {2.0f, 2.0f, 1.0f};
__constant__ float kP4Coef[3][5] = {
    {-0.0020446777f, -0.013000488f, 0.077148438f, -0.06640625f, -0.15429688f},
    {0.0021514893f, -0.0071716309f, -0.0040283203f, 0.063964844f, -0.10009766f},
    {-0.0029296875f, 0.010681152f, -0.015869141f, 0.012023926f, -0.0040283203f},
};

// GELU(x) = relu(x) + q(|x|) with q the 3-piece degree-4 bump, rounded to
// bf16 at exactly the points gelu_poly4_eval.inc rounds. x must already be
// bf16-exact. Returns the fp32 sum before the final rounding.
template <bool RNE>
__device__ __forceinline__ float poly4_gelu_pre(float x) {
  const float s = fabsf(x);
  float q = 0.f;
#pragma unroll
  for (int p = 2; p >= 0; --p) {
    float t = s - kP4Shift[p];
    t = RNE ? rb_rne(t) : rb_trunc(t);
    float u = t * kP4Scale[p];
    u = RNE ? rb_rne(u) : rb_trunc(u);
    float acc = kP4Coef[p][0];
#pragma unroll
    for (int k = 1; k <= 4; ++k) {
      const float ah = RNE ? rb_rne(acc) : rb_trunc(acc);
      // ah * u is exact in fp32 (two bf16 factors), so one rounding
      acc = fmaf(ah, u, kP4Coef[p][k]);
    }
    if (s < kP4Break[p]) q = RNE ? rb_rne(acc) : rb_trunc(acc);
  }
  return fmaxf(x, 0.f) + q;
}

__device__ __forceinline__ uint16_t gelu_variant(float x, int variant) {
  if (variant == GELU_ERF) return f2bf(gelu_erf(x));
  if (variant == GELU_POLY4_RNE) return f2bf(poly4_gelu_pre<true>(rb_rne(x)));
  return f2bf_trunc(poly4_gelu_pre<false>(x));
}

template <int VARIANT, bool XF32>
__global__ __launch_bounds__(256) void gelu_kernel_v8(
    const void* __restrict__ xp, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols8) {
  const int64_t total = (int64_t)rows * cols8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / cols8);
    const int64_t c = (i - (int64_t)r * cols8) * 8;
    float v[8];
    if (XF32) {
      const float* x = static_cast<const float*>(xp) + r * ldx + c;
      f32x4 a = *reinterpret_cast<const f32x4*>(x);
      f32x4 b = *reinterpret_cast<const f32x4*>(x + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[j + 4] = b[j]; }
    } else {
      u16x8 a = *reinterpret_cast<const u16x8*>(
          static_cast<const uint16_t*>(xp) + r * ldx + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = bf2f(a[j]);
    }
    u16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = gelu_variant(v[j], VARIANT);
    *reinterpret_cast<u16x8*>(y + r * ldy + c) = o;
  }
}

template <int VARIANT, bool XF32>
__global__ __launch_bounds__(256) void gelu_kernel_scalar(
    const void* __restrict__ xp, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / cols);
    const int64_t c = i - (int64_t)r * cols;
    const float v = XF32 ? static_cast<const float*>(xp)[r * ldx + c]
                         : bf2f(static_cast<const uint16_t*>(xp)[r * ldx + c]);
    y[r * ldy + c] = gelu_variant(v, VARIANT);
  }
}

static int grid_for(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 256 * 32) g = 256 * 32;
  return (int)(g < 1 ? 1 : g);
}

template <int VARIANT>
static hipError_t gelu_dispatch(const void* x, bool xf, int64_t ldx,
                                uint16_t* y, int64_t ldy, int rows, int cols,
                                hipStream_t s) {
  const size_t xe = xf ? 4 : 2;
  const bool vec = (cols % 8 == 0) && (ldx % 8 == 0) && (ldy % 8 == 0) &&
                   ((uintptr_t)x % (xe * 8 > 16 ? 16 : xe * 8) == 0) &&
                   ((uintptr_t)y % 16 == 0);
  if (vec) {
    const int cols8 = cols / 8;
    const int g = grid_for((int64_t)rows * cols8);
    if (xf)
      gelu_kernel_v8<VARIANT, true><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols8);
    else
      gelu_kernel_v8<VARIANT, false><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols8);
  } else {
    const int g = grid_for((int64_t)rows * cols);
    if (xf)
      gelu_kernel_scalar<VARIANT, true><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols);
    else
      gelu_kernel_scalar<VARIANT, false><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols);
  }
  return hipGetLastError();
}

hipError_t launch_gelu(const void* x, int x_dtype, int64_t ldx, uint16_t* y,
                       int64_t ldy, int rows, int cols, int variant,
                       hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const bool xf = x_dtype == DT_F32;
  switch (variant) {
    case GELU_ERF:
      return gelu_dispatch<GELU_ERF>(x, xf, ldx, y, ldy, rows, cols, s);
    case GELU_POLY4_RNE:
      return gelu_dispatch<GELU_POLY4_RNE>(x, xf, ldx, y, ldy, rows, cols, s);
    case GELU_POLY4_TRUNC:
      return gelu_dispatch<GELU_POLY4_TRUNC>(x, xf, ldx, y, ldy, rows, cols, s);
  }
  return hipErrorInvalidValue;
}

// ======================================================== softmax
// One wave per row, VEC-element chunks held in registers (MAXCH per lane).
template <int VEC, int MAXCH>
__global__ __launch_bounds__(256) void softmax_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols / VEC;
  const uint16_t* xr = x + row * ldx;
  float v[MAXCH][VEC];
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int ch = lane + c * 64;
    if (ch < nch) {
      if (VEC == 8) {
        u16x8 a = *reinterpret_cast<const u16x8*>(xr + ch * 8);
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[c][j] = bf2f(a[j]);
      } else if (VEC == 4) {
        u16x4 a = *reinterpret_cast<const u16x4*>(xr + ch * 4);
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[c][j] = bf2f(a[j]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[c][j] = bf2f(xr[ch * VEC + j]);
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) m = fmaxf(m, v[c][j]);
    }
  }
  m = wave_max(m);
  constexpr float kLog2e = 1.4426950408889634f;
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    if (lane + c * 64 < nch) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        v[c][j] = exp2f((v[c][j] - m) * kLog2e);
        sum += v[c][j];
      }
    }
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  uint16_t* yr = y + row * ldy;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= nch) continue;
    if (VEC == 8) {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = f2bf2(v[c][2 * j] * inv, v[c][2 * j + 1] * inv);
      *reinterpret_cast<u32x4*>(yr + ch * 8) = pk;
    } else if (VEC == 4) {
      u32x2 pk = {f2bf2(v[c][0] * inv, v[c][1] * inv),
                  f2bf2(v[c][2] * inv, v[c][3] * inv)};
      *reinterpret_cast<u32x2*>(yr + ch * 4) = pk;
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) yr[ch * VEC + j] = f2bf(v[c][j] * inv);
    }
  }
}

// Rows wider than the register budget: three passes over global memory.
__global__ __launch_bounds__(256) void softmax_kernel_wide(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * ldx;
  float m = -INFINITY;
  for (int c = lane; c < cols; c += 64) m = fmaxf(m, bf2f(xr[c]));
  m = wave_max(m);
  constexpr float kLog2e = 1.4426950408889634f;
  float sum = 0.f;
  for (int c = lane; c < cols; c += 64) sum += exp2f((bf2f(xr[c]) - m) * kLog2e);
  const float inv = 1.0f / wave_sum(sum);
  uint16_t* yr = y + row * ldy;
  for (int c = lane; c < cols; c += 64)
    yr[c] = f2bf(exp2f((bf2f(xr[c]) - m) * kLog2e) * inv);
}

hipError_t launch_softmax(const uint16_t* x, int64_t ldx, uint16_t* y,
                          int64_t ldy, int rows, int valid, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  dim3 grid((rows + 3) / 4), block(256);
  auto aligned = [&](int vec) {
    return valid % vec == 0 && ldx % vec == 0 && ldy % vec == 0 &&
           (uintptr_t)x % (vec * 2) == 0 && (uintptr_t)y % (vec * 2) == 0;
  };
  if (valid <= 64 * 8 * 8 && aligned(8))
    softmax_kernel<8, 8><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid);
  else if (valid <= 64 * 4 * 16 && aligned(4))
    softmax_kernel<4, 16><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid);
  else if (valid <= 64 * 32)
    softmax_kernel<1, 32><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid);
  else
    softmax_kernel_wide<<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid);
  return hipGetLastError();
}

// ======================================================== conversions
__global__ __launch_bounds__(256) void convert_kernel(
    const float* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / cols);
    const int64_t c = i - (int64_t)r * cols;
    y[r * ldy + c] = f2bf(x[r * ldx + c]);
  }
}

// 64x64 tile transpose through LDS: y[c, r] = bf16(x[r, c]).
__global__ __launch_bounds__(256) void convert_t_kernel(
    const float* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  __shared__ float tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? x[(int64_t)r * ldx + c] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (c < cols && r < rows) y[(int64_t)c * ldy + r] = f2bf(tile[tx][i]);
  }
}

hipError_t launch_convert(const float* x, int64_t ldx, uint16_t* y,
                          int64_t ldy, int rows, int cols, bool transpose,
                          hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (transpose) {
    dim3 grid((cols + 63) / 64, (rows + 63) / 64);
    convert_t_kernel<<<grid, 256, 0, s>>>(x, ldx, y, ldy, rows, cols);
  } else {
    convert_kernel<<<grid_for((int64_t)rows * cols), 256, 0, s>>>(x, ldx, y, ldy,
                                                                   rows, cols);
  }
  return hipGetLastError();
}

// mel [B, C, T] fp32 -> [B, T + 2, C] bf16 with zero edge rows.
__global__ __launch_bounds__(256) void prep_mel_kernel(
    const float* __restrict__ mel, int C, int T, uint16_t* __restrict__ out) {
  __shared__ float tile[64][65];
  const int b = blockIdx.z;
  const int t0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const float* m = mel + (int64_t)b * C * T;
  uint16_t* o = out + (int64_t)b * (T + 2) * C;
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, t = t0 + tx;
    tile[i][tx] = (c < C && t < T) ? m[(int64_t)c * T + t] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int t = t0 + i, c = c0 + tx;
    if (t < T && c < C) o[(int64_t)(t + 1) * C + c] = f2bf(tile[tx][i]);
  }
  if (blockIdx.x == 0) {
    for (int c = c0 + threadIdx.x; c < c0 + 64 && c < C; c += 256) {
      o[c] = 0;
      o[(int64_t)(T + 1) * C + c] = 0;
    }
  }
}

hipError_t launch_prep_mel(const float* mel, int batch, int C, int T,
                           uint16_t* out, hipStream_t s) {
  dim3 grid((T + 63) / 64, (C + 63) / 64, batch);
  prep_mel_kernel<<<grid, 256, 0, s>>>(mel, C, T, out);
  return hipGetLastError();
}

}  // namespace wx
