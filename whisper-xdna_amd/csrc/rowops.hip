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
  // gamma and beta do not depend on the row: their loads are issued first so
  // that their latency overlaps the row load and the two reductions
  f32x4 gb[MAXCH][4];
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int64_t col = (int64_t)(lane + c * 64) * 8;
    const bool ok = lane + c * 64 < nch;
    gb[c][0] = gb[c][1] = f32x4{1.f, 1.f, 1.f, 1.f};
    gb[c][2] = gb[c][3] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (ok && gamma) {
      gb[c][0] = *reinterpret_cast<const f32x4*>(gamma + col);
      gb[c][1] = *reinterpret_cast<const f32x4*>(gamma + col + 4);
    }
    if (ok && beta) {
      gb[c][2] = *reinterpret_cast<const f32x4*>(beta + col);
      gb[c][3] = *reinterpret_cast<const f32x4*>(beta + col + 4);
    }
  }
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
    const f32x4 g0 = gb[c][0], g1 = gb[c][1], b0 = gb[c][2], b1 = gb[c][3];
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

// Rows whose start is not 16-byte aligned (a row pitch that is not a
// multiple of 8 elements, e.g. 1500): the row is read as the 16-byte chunks of
// the aligned span that covers it, chunk c holding elements 8 c - head ..
// 8 c - head + 7 of the row (head = row start mod 8). Only the first and last
// chunk can hold elements outside the row; those are masked to -inf for the
// max and written element by element, every other chunk is one 16-byte load
// and one 16-byte store. Loads go through a buffer descriptor that covers
// exactly the input; the last row's last chunk, the only one that can reach
// past the input's end, is read element by element.
// exp is one FMA and one exp2 per element: p = 2^(x log2e - m log2e + 32)
// / sum; the +32 keeps exp2's result out of the denormal range for every p
// that is representable, and cancels in the division.
template <int MAXCH>
__global__ __launch_bounds__(256) void softmax_kernel_span(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int valid, int x_bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, x_bytes, 0x00020000);
  const int64_t sx = (int64_t)row * ldx, sy = (int64_t)row * ldy;
  const int head = (int)(sx & 7);
  const int64_t ax = sx - head, ay = sy - head;  // ldx == ldy (mod 8): same head
  const int nch = (head + valid + 7) >> 3;
  float v[MAXCH][8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + i * 64;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i][j] = -INFINITY;
    if (c < nch) {
      if (row == rows - 1 && c == nch - 1) {
        // the one chunk that may run past the end of the input: a 16-byte
        // access that crosses the descriptor's range reads as all zeros, so
        // its in-row elements are read one by one
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = c * 8 + j - head;
          if (e >= 0 && e < valid) v[i][j] = bf2f(x[sx + e]);
        }
      } else {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)((ax + c * 8) * 2), 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[i][2 * j] = __uint_as_float(w[j] << 16);
          v[i][2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
      }
      if (c == 0 || c == nch - 1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = c * 8 + j - head;
          if (e < 0 || e >= valid) v[i][j] = -INFINITY;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, v[i][j]);
    }
  }
  m = wave_max(m);
  constexpr float kLog2e = 1.4426950408889634f;
  const float off = 32.0f - m * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    if (lane + i * 64 < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[i][j] = __builtin_amdgcn_exp2f(fmaf(v[i][j], kLog2e, off));
        sum += v[i][j];
      }
    }
  }
  const float inv = 1.0f / wave_sum(sum);
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + i * 64;
    if (c >= nch) continue;
    if (c == 0 || c == nch - 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = c * 8 + j - head;
        if (e >= 0 && e < valid) y[ay + c * 8 + j] = f2bf(v[i][j] * inv);
      }
    } else {
      u32x4 pk;
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = f2bf2(v[i][2 * j] * inv, v[i][2 * j + 1] * inv);
      *reinterpret_cast<u32x4*>(y + ay + c * 8) = pk;
    }
  }
#endif
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
  const int64_t x_bytes = ((int64_t)(rows - 1) * ldx + valid) * 2;
  const bool span = ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
                    (ldx - ldy) % 8 == 0 && x_bytes < (1ll << 31);
  if (valid <= 64 * 8 * 8 && aligned(8))
    softmax_kernel<8, 8><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid);
  else if (span && valid + 7 <= 64 * 8 * 4)
    softmax_kernel_span<4><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid, (int)x_bytes);
  else if (span && valid + 7 <= 64 * 8 * 8)
    softmax_kernel_span<8><<<grid, block, 0, s>>>(x, ldx, y, ldy, rows, valid, (int)x_bytes);
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
