// Symmetric int8 quantisation for the int8 GEMM path, as the reference's
// quantised matmul does it (bench/probe_int8_decode.py:48-74): per-token
// (per-row) scales for activations, per-channel (per output row of W) or
// one per-tensor scale for weights,
//   scale = max|x| / 127   (1 when the row is all zero)
//   q     = rint(x / scale)  (round half to even), as int8.
// The quotient is the correctly rounded fp32 one (quant_quotient: one
// division per row, a corrected product per element), so q and scale equal
// numpy's float32 evaluation bit for bit.
//
// quantize_rows_kernel: one wave per row, the row in registers (NCH chunks
// of 8 per lane), loads through a per-row buffer descriptor (slots past the
// row read zeros, so every load is unconditional and the padding columns
// up to cols_pad come out as zero codes).
// im2col_quant_kernel: the conv front end's im2col rows (kernel 3, padding
// 1), built and quantised per row in one pass: each row has its own scale,
// so the quantised values of one input frame differ between the three rows
// that contain it, and the bf16 path's implicit-GEMM window cannot be used.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace wx {

__device__ __forceinline__ uint32_t pack_q4(float a, float b, float c, float d,
                                            const QuantScale& s) {
  auto q = [&](float x) { return (uint32_t)((int)rintf(quant_quotient(x, s)) & 0xFF); };
  return q(a) | (q(b) << 8) | (q(c) << 16) | (q(d) << 24);
}

// max |v| over the wave (chunks >= nch hold zeros), then 127ths
__device__ __forceinline__ float row_scale(float m) {
  m = wave_max(m);
  const float s = m / 127.0f;
  return s == 0.f ? 1.0f : s;
}

// Rows are read once: the loads carry the non-temporal hint (cache-policy
// bit 1), which keeps large activations (fc2's 491 MB fp32 A at batch 16)
// from displacing what the next GEMM reads.
constexpr int kCpolNt = 2;

template <int NCH, bool XF32>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const void* __restrict__ xp, int64_t ldx, int rows, int cols, int8_t* __restrict__ q,
    int64_t ldq, int cols_pad, float* __restrict__ scale, int given) {
  const int lane = threadIdx.x & 63;
  const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= rows) return;
  constexpr int esz = XF32 ? 4 : 2;
  const int nbytes = __builtin_amdgcn_readfirstlane(cols * esz);
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(xp) + row * ldx * esz), (short)0, nbytes,
      0x00020000);
  // fp32 rows are read as lane-contiguous 16-byte pieces: v[c][4k .. 4k + 3]
  // are columns col_of(c, k) .. + 3, so one load instruction covers 1 KB of
  // the row (8-column chunks per lane would take two half-used 2 KB spans);
  // bf16 rows keep 8-column chunks, one 16-byte piece per lane
  auto col_of = [&](int c, int k) {
    return XF32 ? ((2 * c + k) * 64 + lane) * 4 : (lane + c * 64) * 8 + 4 * k;
  };
  float v[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (XF32) {
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, col_of(c, 0) * 4, 0, kCpolNt);
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rs, col_of(c, 1) * 4, 0, kCpolNt);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][j] = __uint_as_float(a[j]);
        v[c][j + 4] = __uint_as_float(b[j]);
      }
    } else {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, col_of(c, 0) * 2, 0, kCpolNt);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][2 * j] = __uint_as_float(w[j] << 16);
        v[c][2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
      }
    }
  }
  float s;
  if (given) {
    s = scale[0];
  } else {
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[c][j]));
    s = row_scale(m);
    if (lane == 0) scale[row] = s;
  }
  int8_t* qr = q + row * ldq;
  const QuantScale qs = quant_scale(s);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (XF32) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (col_of(c, k) < cols_pad)
          *reinterpret_cast<uint32_t*>(qr + col_of(c, k)) =
              pack_q4(v[c][4 * k], v[c][4 * k + 1], v[c][4 * k + 2], v[c][4 * k + 3], qs);
    } else if (col_of(c, 0) < cols_pad) {
      const u32x2 o = {pack_q4(v[c][0], v[c][1], v[c][2], v[c][3], qs),
                       pack_q4(v[c][4], v[c][5], v[c][6], v[c][7], qs)};
      *reinterpret_cast<u32x2*>(qr + col_of(c, 0)) = o;
    }
  }
}

hipError_t launch_quantize_rows(const void* x, int x_dtype, int64_t ldx, int rows, int cols,
                                int8_t* q, int64_t ldq, int cols_pad, float* scale,
                                bool given, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const dim3 grid((rows + 3) / 4), block(256);
  const bool xf = x_dtype == DT_F32;
  switch ((cols_pad + 511) / 512) {
#define WX_Q(N)                                                                         \
  case N:                                                                               \
    if (xf)                                                                             \
      quantize_rows_kernel<N, true><<<grid, block, 0, s>>>(x, ldx, rows, cols, q, ldq,  \
                                                           cols_pad, scale, given);     \
    else                                                                                \
      quantize_rows_kernel<N, false><<<grid, block, 0, s>>>(x, ldx, rows, cols, q, ldq, \
                                                            cols_pad, scale, given);    \
    return hipGetLastError();
    WX_Q(1) WX_Q(2) WX_Q(3) WX_Q(4) WX_Q(5) WX_Q(6) WX_Q(7) WX_Q(8)
    WX_Q(9) WX_Q(10) WX_Q(11) WX_Q(12) WX_Q(13) WX_Q(14) WX_Q(15) WX_Q(16)
#undef WX_Q
  }
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------ per-tensor scale
// out (as uint bits) <- max over the band of |x|'s bits: for non-negative
// floats the bit patterns order like the values. Three launches: clear,
// reduce (block max, one atomic per block), finish (bits -> max / 127).
__global__ void absmax_clear_kernel(unsigned* bits) { *bits = 0u; }

template <bool XF32>
__global__ __launch_bounds__(256) void absmax_kernel(const void* __restrict__ xp, int64_t ldx,
                                                     int rows, int cols,
                                                     unsigned* __restrict__ bits) {
  __shared__ float red[4];
  float m = 0.f;
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / cols);
    const int64_t c = i - (int64_t)r * cols;
    const float v = XF32 ? static_cast<const float*>(xp)[r * ldx + c]
                         : bf2f(static_cast<const uint16_t*>(xp)[r * ldx + c]);
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    atomicMax(bits, __float_as_uint(m));
  }
}

__global__ void absmax_finish_kernel(const unsigned* bits, float* out) {
  const float s = __uint_as_float(*bits) / 127.0f;
  *out = s == 0.f ? 1.0f : s;
}

hipError_t launch_absmax_scale(const void* x, int x_dtype, int64_t ldx, int rows, int cols,
                               float* out, unsigned* scratch, hipStream_t s) {
  absmax_clear_kernel<<<1, 1, 0, s>>>(scratch);
  const int64_t work = (int64_t)rows * cols;
  const int g = (int)std::max<int64_t>(1, std::min<int64_t>((work + 255) / 256, 2048));
  if (work > 0) {
    if (x_dtype == DT_F32)
      absmax_kernel<true><<<g, 256, 0, s>>>(x, ldx, rows, cols, scratch);
    else
      absmax_kernel<false><<<g, 256, 0, s>>>(x, ldx, rows, cols, scratch);
  }
  absmax_finish_kernel<<<1, 1, 0, s>>>(scratch, out);
  return hipGetLastError();
}

// ------------------------------------------------------------ conv im2col
// Output row (b, t), t < T_out: K = 3 C values, tap-major (k = j C + c holds
// x[b, stride t - 1 + j, c], zero outside [0, T_in)), then zeros up to ldq.
// One wave per row; C % 8 == 0, so a chunk of 8 never straddles two taps.
template <int NCH>
__global__ __launch_bounds__(256) void im2col_quant_kernel(const float* __restrict__ x,
                                                           int batch, int T_in, int C,
                                                           int stride, int T_out,
                                                           int8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= batch * T_out) return;
  const int b = row / T_out, t = row - b * T_out;
  const int K = 3 * C;
  float v[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = (lane + c * 64) * 8;
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    if (k < K) {
      const int j = k / C, ch = k - j * C;
      const int src = stride * t - 1 + j;
      if (src >= 0 && src < T_in) {
        const f32x4* p = reinterpret_cast<const f32x4*>(x + ((int64_t)b * T_in + src) * C + ch);
        lo = p[0];
        hi = p[1];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[c][r] = lo[r];
      v[c][r + 4] = hi[r];
    }
  }
  float m = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[c][j]));
  const float s = row_scale(m);
  if (lane == 0) scale[row] = s;
  int8_t* qr = q + row * ldq;
  const int npc = (int)(ldq >> 3);
  const QuantScale qs = quant_scale(s);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= npc) continue;
    const u32x2 o = {pack_q4(v[c][0], v[c][1], v[c][2], v[c][3], qs),
                     pack_q4(v[c][4], v[c][5], v[c][6], v[c][7], qs)};
    *reinterpret_cast<u32x2*>(qr + ch * 8) = o;
  }
}

hipError_t launch_im2col_quant(const float* x, int batch, int T_in, int C, int stride,
                               int T_out, int8_t* q, int64_t ldq, float* scale,
                               hipStream_t s) {
  const int rows = batch * T_out;
  if (rows <= 0) return hipSuccess;
  const dim3 grid((rows + 3) / 4), block(256);
  switch ((int)((ldq + 511) / 512)) {
#define WX_IC(N)                                                                      \
  case N:                                                                             \
    im2col_quant_kernel<N><<<grid, block, 0, s>>>(x, batch, T_in, C, stride, T_out, q, \
                                                  ldq, scale);                        \
    return hipGetLastError();
    WX_IC(1) WX_IC(2) WX_IC(3) WX_IC(4) WX_IC(5) WX_IC(6) WX_IC(7) WX_IC(8)
#undef WX_IC
  }
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------ transpose
// [B, C, T] -> [B, T, C], 64 x 64 tiles through LDS
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ x, int C,
                                                            int T, float* __restrict__ y) {
  __shared__ float tile[64][65];
  const int b = blockIdx.z;
  const int t0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const float* xb = x + (int64_t)b * C * T;
  float* yb = y + (int64_t)b * T * C;
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, t = t0 + tx;
    tile[i][tx] = (c < C && t < T) ? xb[(int64_t)c * T + t] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int t = t0 + i, c = c0 + tx;
    if (t < T && c < C) yb[(int64_t)t * C + c] = tile[tx][i];
  }
}

hipError_t launch_transpose_f32(const float* x, int batch, int C, int T, float* y,
                                hipStream_t s) {
  if (batch <= 0 || C <= 0 || T <= 0) return hipSuccess;
  const dim3 grid((T + 63) / 64, (C + 63) / 64, batch);
  transpose_f32_kernel<<<grid, 256, 0, s>>>(x, C, T, y);
  return hipGetLastError();
}

}  // namespace wx
