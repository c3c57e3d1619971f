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
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace wx {

// ======================================================== LayerNorm
// One wave per row; lane l owns 8-element chunks l, l+64, ... of the row
// (NCH = chunks per lane, the row width rounded up to 512). A wave walks
// rows row0, row0 + waves, ...: the next row's loads are issued before the
// current row's reductions, so each wave keeps a row in flight while it
// computes. gamma and beta (or 1 and 0) sit in LDS, loaded once per
// workgroup. STREAM puts the non-temporal hint on the row loads and the
// output stores (standalone calls: nothing reads the rows again soon); NTL
// on the row loads only (see launch_layernorm).
template <int NCH, bool XF32, bool RESID, bool STREAM, bool NTL = false>
struct LnRow {
  // Quad layout: fp32 rows without a residual are loaded as lane-contiguous
  // 16-byte pieces, chunk slot c holding columns (128c + lane) * 4 .. + 3
  // and (128c + 64 + lane) * 4 .. + 3, so that one load instruction covers
  // 1 KB of the row (the 8-column chunks take two half-used 2 KB spans).
  // Measured on the fp32 [24000, 1280] -> bf16 LayerNorm: 35.5 -> 32.7 us.
  static constexpr bool QL = XF32 && !RESID;
  u32x4 x[NCH][XF32 ? 2 : 1];
  u32x4 r[NCH][RESID ? 2 : 1];
  // Every chunk slot is loaded through a descriptor that covers exactly the
  // row (row is wave-uniform), so slots past the row read zeros instead of
  // faulting: the loads are unconditional and their count is the same on
  // every path, which lets the next row's loads stay in flight.
  // A row outside [0, rows) gets an empty descriptor: its loads return
  // zeros without touching memory, and are still issued.
  // cols4 = the row's width in fp32 bytes (4 cols), computed once by the
  // kernel in scalar registers
  __device__ __forceinline__ void load(const void* xp, int64_t ldx, const float* rp,
                                       int64_t ldr, int row, int rows, int lane, int cols4) {
    constexpr int esz = XF32 ? 4 : 2;
    constexpr int aux = STREAM || NTL ? 2 : 0;  // cache-policy bit 1: non-temporal
    const bool in = row < rows;
    row = in ? row : 0;
    const int nx = in ? (XF32 ? cols4 : cols4 >> 1) : 0;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(xp) + row * ldx * esz), (short)0, nx,
        0x00020000);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int h = 0; h < (XF32 ? 2 : 1); ++h)
        x[c][h] = __builtin_amdgcn_raw_buffer_load_b128(
            rs, QL ? ((2 * c + h) * 64 + lane) * 16 : (lane + c * 64) * 8 * esz + h * 16, 0,
            aux);
    if (RESID) {
      const int nr = in ? cols4 : 0;
      const auto rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rp + row * ldr),
                                                        (short)0, nr, 0x00020000);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          r[c][RESID ? h : 0] =
              __builtin_amdgcn_raw_buffer_load_b128(rr, (lane + c * 64) * 32 + h * 16, 0, aux);
    }
  }
};

// LayerNorm of one row from its loaded chunks; gb = gamma [cols], beta [cols].
// YT: DT_BF16, DT_F32, or DT_I8 (the fp32 result quantised per row:
// scale = max|y| / 127, or 1 for an all-zero row, q = rint(y / scale); the
// scale goes to ysc[row])
template <int NCH, bool XF32, int YT, bool RESID, bool STREAM, bool NTL>
__device__ __forceinline__ void ln_row(const LnRow<NCH, XF32, RESID, STREAM, NTL>& cur,
                                       const float* gb, float* __restrict__ sp, int64_t lds,
                                       float eps, void* __restrict__ yp, int64_t ldy, int row,
                                       int lane, int cols, float* __restrict__ ysc) {
  auto st = [](auto v, auto* p) {
    if (STREAM) __builtin_nontemporal_store(v, p); else *p = v;
  };
  const int nch = cols >> 3;
  const float inv_n = 1.0f / (float)cols;
  // v[c][4k .. 4k + 3] are columns col_of(c, k) .. + 3: adjacent halves of
  // the 8-column chunk lane + 64c, or the quad layout's two runs
  constexpr bool QL = LnRow<NCH, XF32, RESID, STREAM>::QL;
  auto col_of = [&](int c, int k) {
    return QL ? ((2 * c + k) * 64 + lane) * 4 : (lane + c * 64) * 8 + 4 * k;
  };
  float v[NCH][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = lane + c * 64;
    if (XF32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][j] = __uint_as_float(cur.x[c][0][j]);
        v[c][j + 4] = __uint_as_float(cur.x[c][XF32 ? 1 : 0][j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][2 * j] = __uint_as_float(cur.x[c][0][j] << 16);
        v[c][2 * j + 1] = __uint_as_float(cur.x[c][0][j] & 0xFFFF0000u);
      }
    }
    if (RESID) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[c][j] += __uint_as_float(cur.r[c][0][j]);
        v[c][j + 4] += __uint_as_float(cur.r[c][RESID ? 1 : 0][j]);
      }
      if (sp && ch < nch) {
        float* o = sp + row * lds + (int64_t)ch * 8;
        st(f32x4{v[c][0], v[c][1], v[c][2], v[c][3]}, reinterpret_cast<f32x4*>(o));
        st(f32x4{v[c][4], v[c][5], v[c][6], v[c][7]}, reinterpret_cast<f32x4*>(o + 4));
      }
    }
    // slots past the row loaded zeros: they add nothing to the sum
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[c][j];
  }
  const float mean = wave_sum(sum) * inv_n;
  // second pass over the registers: exact two-pass variance
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (col_of(c, k) < cols) {
#pragma unroll
        for (int j = 4 * k; j < 4 * k + 4; ++j) {
          const float dlt = v[c][j] - mean;
          sq += dlt * dlt;
        }
      }
    }
  }
  const float var = wave_sum(sq) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
  if constexpr (YT == DT_I8) {
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int col = col_of(c, k);
        if (col >= cols) continue;
        const f32x4 g = *reinterpret_cast<const f32x4*>(gb + col);
        const f32x4 bb = *reinterpret_cast<const f32x4*>(gb + cols + col);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[c][4 * k + j] = (v[c][4 * k + j] - mean) * rstd * g[j] + bb[j];
          m = fmaxf(m, fabsf(v[c][4 * k + j]));
        }
      }
    }
    m = wave_max(m) / 127.0f;
    const float sc = m == 0.f ? 1.0f : m;
    if (lane == 0) ysc[row] = sc;
    const QuantScale qs = quant_scale(sc);
    auto q4 = [&](const float* a) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w |= (uint32_t)((int)rintf(quant_quotient(a[j], qs)) & 0xFF) << (8 * j);
      return w;
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      int8_t* y = static_cast<int8_t*>(yp) + row * ldy;
      if (!QL) {
        if (col_of(c, 0) < cols)
          st(u32x2{q4(&v[c][0]), q4(&v[c][4])}, reinterpret_cast<u32x2*>(y + col_of(c, 0)));
        continue;
      }
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (col_of(c, k) < cols)
          st(q4(&v[c][4 * k]), reinterpret_cast<uint32_t*>(y + col_of(c, k)));
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float o[8];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int col = col_of(c, k) < cols ? col_of(c, k) : 0;
      const f32x4 g = *reinterpret_cast<const f32x4*>(gb + col);
      const f32x4 bb = *reinterpret_cast<const f32x4*>(gb + cols + col);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[4 * k + j] = (v[c][4 * k + j] - mean) * rstd * g[j] + bb[j];
    }
    if (YT == DT_F32) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (col_of(c, k) < cols)
          st(f32x4{o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]},
             reinterpret_cast<f32x4*>(static_cast<float*>(yp) + row * ldy + col_of(c, k)));
    } else if (!QL) {
      if (col_of(c, 0) < cols)
        st(u32x4{f2bf2(o[0], o[1]), f2bf2(o[2], o[3]), f2bf2(o[4], o[5]), f2bf2(o[6], o[7])},
           reinterpret_cast<u32x4*>(static_cast<uint16_t*>(yp) + row * ldy + col_of(c, 0)));
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (col_of(c, k) < cols)
          st(u32x2{f2bf2(o[4 * k], o[4 * k + 1]), f2bf2(o[4 * k + 2], o[4 * k + 3])},
             reinterpret_cast<u32x2*>(static_cast<uint16_t*>(yp) + row * ldy + col_of(c, k)));
    }
  }
}

template <int NCH, bool XF32, int YT, bool RESID, bool STREAM, bool NTL = false>
__global__ __launch_bounds__(256) void ln_kernel(
    const void* __restrict__ xp, int64_t ldx, const float* __restrict__ rp,
    int64_t ldr, float* __restrict__ sp, int64_t lds,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    void* __restrict__ yp, int64_t ldy, int rows, int cols, float* __restrict__ ysc) {
  extern __shared__ __align__(16) float ln_gb[];  // gamma [cols], beta [cols]
  // wave-uniform; readfirstlane keeps it (and the descriptor lengths made
  // from it) in scalar registers: cols is also read in the divergent loop
  // below, after which the compiler would hold it in a VGPR
  const int cols4 = __builtin_amdgcn_readfirstlane(cols * 4);
  const int lane = threadIdx.x & 63;
  const int row0 = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int waves = gridDim.x * 4;
  // two row buffers in turn (no register copies, which would wait for the
  // loads in flight); the first row's loads go out before gamma and beta
  // are fetched, so the two trips to memory overlap
  LnRow<NCH, XF32, RESID, STREAM, NTL> ra, rb;
  int row = row0;
  ra.load(xp, ldx, rp, ldr, row, rows, lane, cols4);
  {
    // gamma and beta as 16-byte pieces (cols <= 4096: at most 4 per thread),
    // every load issued before the LDS writes
    // (unconditional buffer loads: past the end, or for a null gamma or
    // beta, they read zeros; a null gamma then becomes ones)
    constexpr int kPer = kMaxRowCols / 4 / 256;
    const int n4 = cols >> 2;
    const auto rg = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(gamma), (short)0,
                                                      gamma ? cols4 : 0, 0x00020000);
    const auto rb2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(beta), (short)0,
                                                       beta ? cols4 : 0, 0x00020000);
    u32x4 g[kPer], b[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int off = (threadIdx.x + k * 256) * 16;
      g[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0);
      b[k] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = threadIdx.x + k * 256;
      if (i < n4) {
        reinterpret_cast<u32x4*>(ln_gb)[i] =
            gamma ? g[k] : u32x4{0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u};
        reinterpret_cast<u32x4*>(ln_gb + cols)[i] = b[k];
      }
    }
  }
  __syncthreads();
  while (row < rows) {
    rb.load(xp, ldx, rp, ldr, row + waves, rows, lane, cols4);
    ln_row<NCH, XF32, YT, RESID, STREAM, NTL>(ra, ln_gb, sp, lds, eps, yp, ldy, row, lane,
                                              cols, ysc);
    row += waves;
    if (row >= rows) break;
    ra.load(xp, ldx, rp, ldr, row + waves, rows, lane, cols4);
    ln_row<NCH, XF32, YT, RESID, STREAM, NTL>(rb, ln_gb, sp, lds, eps, yp, ldy, row, lane,
                                              cols, ysc);
    row += waves;
  }
}

// Workgroups at most: 2048 waves, each walking ~rows / 2048 rows with the
// next row in flight (512 measured best at the encoder's [24000, 1280]).
constexpr int kLnGrid = 512;

template <int NCH>
static hipError_t ln_dispatch(const void* x, int x_dtype, int64_t ldx,
                              const float* resid, int64_t ldr, float* sum_out,
                              int64_t lds, const float* gamma,
                              const float* beta, float eps, void* y,
                              int y_dtype, int64_t ldy, int rows, int cols,
                              bool stream, bool ntl, hipStream_t s, float* ysc) {
  dim3 grid(std::min((rows + 3) / 4, kLnGrid)), block(256);
  const size_t smem = 2 * (size_t)cols * sizeof(float);
  const bool xf = x_dtype == DT_F32, r = resid != nullptr;
  const int yt = y_dtype;
#define WX_LN_NTL(YT)                                                                  \
  if (ntl)                                                                             \
    ln_kernel<NCH, true, YT, false, false, true><<<grid, block, smem, s>>>(            \
        x, ldx, resid, ldr, sum_out, lds, gamma, beta, eps, y, ldy, rows, cols, ysc);   \
  else                                                                                 \
    ln_kernel<NCH, true, YT, false, false, false><<<grid, block, smem, s>>>(           \
        x, ldx, resid, ldr, sum_out, lds, gamma, beta, eps, y, ldy, rows, cols, ysc);   \
  return hipGetLastError();
  if (yt == DT_I8) {
    // the int8 encoder's LayerNorm only: fp32 residual stream in, no fused
    // residual add, cached stores
    if (!xf || r || stream) return hipErrorInvalidValue;
    WX_LN_NTL(DT_I8)
  }
  // the encoder's LayerNorm (fp32 residual stream in, cached stores)
  if (xf && !r && !stream && yt == DT_BF16) { WX_LN_NTL(DT_BF16) }
#undef WX_LN_NTL
#define WX_LN(XF, YT, R)                                                             \
  if (xf == XF && yt == YT && r == R) {                                              \
    if (stream)                                                                      \
      ln_kernel<NCH, XF, YT, R, true><<<grid, block, smem, s>>>(                     \
          x, ldx, resid, ldr, sum_out, lds, gamma, beta, eps, y, ldy, rows, cols, ysc); \
    else                                                                             \
      ln_kernel<NCH, XF, YT, R, false><<<grid, block, smem, s>>>(                    \
          x, ldx, resid, ldr, sum_out, lds, gamma, beta, eps, y, ldy, rows, cols, ysc); \
    return hipGetLastError();                                                        \
  }
  WX_LN(false, DT_BF16, false) WX_LN(false, DT_F32, false)
  WX_LN(true, DT_BF16, false) WX_LN(true, DT_F32, false)
  WX_LN(false, DT_BF16, true) WX_LN(false, DT_F32, true)
  WX_LN(true, DT_BF16, true) WX_LN(true, DT_F32, true)
#undef WX_LN
  return hipErrorInvalidValue;
}

hipError_t launch_layernorm(const void* x, int x_dtype, int64_t ldx,
                            const float* resid, int64_t ldr, float* sum_out,
                            int64_t lds, const float* gamma, const float* beta,
                            float eps, void* y, int y_dtype, int64_t ldy,
                            int rows, int cols, bool stream, hipStream_t s,
                            float* y_scale) {
  if (rows <= 0) return hipSuccess;
  // The encoder's LayerNorm (cached stores: the next GEMM reads its output)
  // loads a large fp32 residual stream with the non-temporal hint, so that
  // the stream does not push the GEMMs' operands out of L2 and the Infinity
  // Cache: batch-16 large-v3 forward 38.62 -> 38.45 ms, int8 34.63 ->
  // 34.34. A small one is still in the Infinity Cache when the residual
  // GEMM that follows reads it again, and the hint costs that reuse (batch 1:
  // 4.19 -> 4.26 ms; at 42 MB, batch 16 at ctx 512, 15.50 -> 15.55 ms).
  // Between the two reads the stream, the LayerNorm's output and the QKV
  // and attention outputs come to 3.5 times the stream; the switch sits at
  // 64 MB, where that is 224 of the cache's 256 MB.
  const bool ntl = !stream && x_dtype == DT_F32 && !resid &&
                   (int64_t)rows * cols * 4 >= (int64_t)64 << 20;
  // chunks of 8 per lane: 64 lanes x 8 = 512 columns per chunk
  switch ((cols + 511) / 512) {
#define WX_LNC(N)                                                                   \
    case N:                                                                         \
      return ln_dispatch<N>(x, x_dtype, ldx, resid, ldr, sum_out, lds, gamma, beta, \
                            eps, y, y_dtype, ldy, rows, cols, stream, ntl, s, y_scale);
    WX_LNC(1) WX_LNC(2) WX_LNC(3) WX_LNC(4) WX_LNC(5) WX_LNC(6) WX_LNC(7) WX_LNC(8)
#undef WX_LNC
  }
  return hipErrorInvalidValue;
}

// ======================================================== GELU
// The standalone GELU streams: every element is read once and written once,
// so the loads and stores carry the non-temporal hint (the data is not
// wanted in L2 or the Infinity Cache afterwards; on this GPU that lifts a
// plain copy of the [1500, 5120] bf16 rowops shape from 3.9 to 5.2 TB/s).
// A thread handles kGeluChunks 16-byte chunks per trip, loads first, then
// math and stores.
//
// poly4 GELU with RNE (g4r, and g4f after its input rounding) by table: for
// a bf16 input, the bump q of poly4_q depends only on the bit pattern of
// |x|. At or below 2^-10 (pattern 0x3A80), rb(|x| - 0.5) is -0.5 (the tie
// at 2^-10 goes to the even -0.5), so q equals q(0); from 4.0 (0x4080) up,
// and for inf and NaN, q is 0. g_poly4_q holds q for the patterns
// 0x3A80 .. 0x4080, written once per device by poly4_table_kernel from
// poly4_q itself, so the table path returns the arithmetic path's bits; a
// GELU workgroup copies it (3 KB) to LDS and looks q up by the pattern
// clamped into that range: 9 operations and one LDS read per element in
// place of ~35. The truncating variant (g4) keeps the arithmetic: under
// truncation q is not constant below 2^-9.
constexpr int kP4LutBase = 0x3A80;
constexpr int kP4LutLen = 0x4080 - kP4LutBase + 1;      // 1537
constexpr int kP4LutPad = (kP4LutLen + 7) / 8 * 8;      // 16-byte multiple
__device__ __align__(16) uint16_t g_poly4_q[kP4LutPad];

__global__ __launch_bounds__(256) void poly4_table_kernel() {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < kP4LutPad)
    g_poly4_q[i] = i < kP4LutLen ? f2bf(poly4_q<true>(bf2f((uint16_t)(kP4LutBase + i)))) : 0;
}

hipError_t init_rowop_tables(hipStream_t s) {
  poly4_table_kernel<<<(kP4LutPad + 255) / 256, 256, 0, s>>>();
  return hipGetLastError();
}

// poly4 GELU (RNE) of a bf16-exact x, q looked up in the LDS copy of the
// table: the pattern of |x| clamped into [0x3A80, 0x4080] (v_med3_i32)
__device__ __forceinline__ float poly4_gelu_lut(float x, const uint16_t* lut) {
  const int bits = (int)(__float_as_uint(x) >> 16) & 0x7FFF;
  const int idx = min(max(bits - kP4LutBase, 0), kP4LutLen - 1);
  return fmaxf(x, 0.f) + bf2f(lut[idx]);
}

template <int VARIANT>
__device__ __forceinline__ uint32_t gelu_pair(float a, float b, const uint16_t* lut) {
  if (VARIANT == GELU_ERF) return f2bf2(gelu_erf(a), gelu_erf(b));
  if (VARIANT == GELU_POLY4_RNE)
    return f2bf2(poly4_gelu_lut(rb_rne(a), lut), poly4_gelu_lut(rb_rne(b), lut));
  return (uint32_t)f2bf_trunc(poly4_gelu_pre<false>(a)) |
         ((uint32_t)f2bf_trunc(poly4_gelu_pre<false>(b)) << 16);
}

// 16-byte chunks per thread per trip, and workgroups at most: the whole
// grid for erf (one trip each), 1024 for the table variant, whose
// workgroups each copy the 3 KB table first (measured on [1500, 5120]).
constexpr int kGeluChunks = 2;
constexpr int kGeluGridErf = 1 << 20, kGeluGridLut = 1024;

// 8-element chunks i in [0, total8): chunk i is row i / cols8, columns
// 8 (i % cols8) .. + 7 (CONTIG: the rows are packed, offset 8 i). The host
// keeps total8 + the grid's stride below 2^32.
template <int VARIANT, bool XF32, bool CONTIG, int CH>
__global__ __launch_bounds__(256) void gelu_kernel_v8(
    const void* __restrict__ xp, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, uint32_t cols8, uint32_t total8) {
  constexpr bool kLut = VARIANT == GELU_POLY4_RNE;
  __shared__ __align__(16) uint16_t lut[kLut ? kP4LutPad : 8];
  if (kLut) {
    for (int i = threadIdx.x; i < kP4LutPad / 8; i += 256)
      reinterpret_cast<u32x4*>(lut)[i] = reinterpret_cast<const u32x4*>(g_poly4_q)[i];
    __syncthreads();
  }
  const uint32_t stride = gridDim.x * (256u * CH);
  for (uint32_t base = blockIdx.x * (256u * CH) + threadIdx.x; base < total8;
       base += stride) {
    float v[CH][8];
    int64_t oy[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const uint32_t i = base + j * 256u;
      if (i >= total8) continue;
      int64_t ox;
      if (CONTIG) {
        ox = oy[j] = (int64_t)i * 8;
      } else {
        const uint32_t r = i / cols8, c = (i - r * cols8) * 8;
        ox = r * ldx + c;
        oy[j] = r * ldy + c;
      }
      if (XF32) {
        const f32x4* x = reinterpret_cast<const f32x4*>(static_cast<const float*>(xp) + ox);
        const f32x4 a = __builtin_nontemporal_load(x), b = __builtin_nontemporal_load(x + 1);
#pragma unroll
        for (int k = 0; k < 4; ++k) { v[j][k] = a[k]; v[j][k + 4] = b[k]; }
      } else {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            static_cast<const uint16_t*>(xp) + ox));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[j][2 * k] = __uint_as_float(w[k] << 16);
          v[j][2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (base + j * 256u >= total8) continue;
      u32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = gelu_pair<VARIANT>(v[j][2 * k], v[j][2 * k + 1], lut);
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(y + oy[j]));
    }
  }
}

__device__ __forceinline__ uint16_t gelu_variant(float x, int variant, const uint16_t* lut) {
  if (variant == GELU_ERF) return f2bf(gelu_erf(x));
  if (variant == GELU_POLY4_RNE) return f2bf(poly4_gelu_lut(rb_rne(x), lut));
  return f2bf_trunc(poly4_gelu_pre<false>(x));
}

// Any alignment and width, one element per thread and trip.
template <int VARIANT, bool XF32>
__global__ __launch_bounds__(256) void gelu_kernel_scalar(
    const void* __restrict__ xp, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int cols) {
  constexpr bool kLut = VARIANT == GELU_POLY4_RNE;
  __shared__ __align__(16) uint16_t lut[kLut ? kP4LutPad : 8];
  if (kLut) {
    for (int i = threadIdx.x; i < kP4LutPad / 8; i += 256)
      reinterpret_cast<u32x4*>(lut)[i] = reinterpret_cast<const u32x4*>(g_poly4_q)[i];
    __syncthreads();
  }
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / cols);
    const int64_t c = i - (int64_t)r * cols;
    const float v = XF32 ? static_cast<const float*>(xp)[r * ldx + c]
                         : bf2f(static_cast<const uint16_t*>(xp)[r * ldx + c]);
    y[r * ldy + c] = gelu_variant(v, VARIANT, lut);
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
                   ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
  if (!vec) {
    const int g = grid_for((int64_t)rows * cols);
    if (xf)
      gelu_kernel_scalar<VARIANT, true><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols);
    else
      gelu_kernel_scalar<VARIANT, false><<<g, 256, 0, s>>>(x, ldx, y, ldy, rows, cols);
    return hipGetLastError();
  }
  const uint32_t cols8 = (uint32_t)(cols / 8);
  const bool contig = ldx == cols && ldy == cols;
  // row bands of at most 2^30 chunks keep every 32-bit chunk index (plus
  // the grid's stride) below 2^32
  const int band = (int)std::min<int64_t>(rows, (int64_t)(1u << 30) / cols8);
  for (int r0 = 0; r0 < rows; r0 += band) {
    const int nr = std::min(band, rows - r0);
    const uint32_t total8 = (uint32_t)nr * cols8;
    constexpr int cap = VARIANT == GELU_POLY4_RNE ? kGeluGridLut : kGeluGridErf;
    const int g = (int)std::min<int64_t>((total8 + 256 * kGeluChunks - 1) / (256 * kGeluChunks),
                                         cap);
    const void* xb = static_cast<const char*>(x) + (int64_t)r0 * ldx * xe;
    uint16_t* yb = y + (int64_t)r0 * ldy;
#define WX_GELU(XF, CG)                                                     \
    if (xf == XF && contig == CG)                                           \
      gelu_kernel_v8<VARIANT, XF, CG, kGeluChunks><<<g, 256, 0, s>>>(xb, ldx, yb, ldy, cols8, \
                                                                    total8);
    WX_GELU(true, true) WX_GELU(true, false) WX_GELU(false, true) WX_GELU(false, false)
#undef WX_GELU
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
// Rows are read once and written once: loads and stores carry the
// non-temporal hint (buffer loads: cache-policy bit 1, NT on this GPU).
constexpr int kCpolNt = 2;
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
        u16x8 a = __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(xr + ch * 8));
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[c][j] = bf2f(a[j]);
      } else if (VEC == 4) {
        u16x4 a = __builtin_nontemporal_load(reinterpret_cast<const u16x4*>(xr + ch * 4));
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
      __builtin_nontemporal_store(pk, reinterpret_cast<u32x4*>(yr + ch * 8));
    } else if (VEC == 4) {
      u32x2 pk = {f2bf2(v[c][0] * inv, v[c][1] * inv),
                  f2bf2(v[c][2] * inv, v[c][3] * inv)};
      __builtin_nontemporal_store(pk, reinterpret_cast<u32x2*>(yr + ch * 4));
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
// One row's MAXCH chunk slots per lane, loaded unconditionally: a slot past
// the row's last chunk gets an offset beyond the descriptor's range, so it
// reads zeros without touching memory (the row math masks it). Not for the
// last row, whose last chunk may cross the end of the input.
constexpr uint32_t kOutOfRange = 0x80000000u;  // > any x_bytes (< 2^31)
template <int MAXCH>
__device__ __forceinline__ void softmax_span_load(u32x4 (&w)[MAXCH], __amdgpu_buffer_rsrc_t rx,
                                                  int64_t sx, int lane, int nch) {
  const uint32_t a = (uint32_t)((sx & ~(int64_t)7) * 2);
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + i * 64;
    const uint32_t off = c < nch ? a + (uint32_t)c * 16 : kOutOfRange;
    w[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, kCpolNt);
  }
}

// The last row: the chunk that can run past the end of the input is read
// element by element (a 16-byte access that crosses the descriptor's range
// reads as all zeros).
template <int MAXCH>
__device__ __forceinline__ void softmax_span_load_last(u32x4 (&w)[MAXCH], __amdgpu_buffer_rsrc_t rx,
                                                       const uint16_t* __restrict__ x, int64_t sx,
                                                       int lane, int valid) {
  const int head = (int)(sx & 7);
  const int nch = (head + valid + 7) >> 3;
  softmax_span_load<MAXCH>(w, rx, sx, lane, nch);
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + i * 64;
    if (c != nch - 1) continue;
    uint32_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = c * 8 + j - head;
      e[j] = (k >= 0 && k < valid) ? x[sx + k] : 0u;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) w[i][j] = e[2 * j] | (e[2 * j + 1] << 16);
  }
}

// softmax of one row from its loaded chunks; stores to y
template <int MAXCH>
__device__ __forceinline__ void softmax_span_row(const u32x4 (&w)[MAXCH], uint16_t* __restrict__ y,
                                                 int64_t sx, int64_t sy, int lane, int valid) {
  constexpr float kLog2e = 1.4426950408889634f;
  const int head = (int)(sx & 7);
  const int64_t ay = sy - head;  // ldx == ldy (mod 8): same head
  const int nch = (head + valid + 7) >> 3;
  float v[MAXCH][8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int c = lane + i * 64;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][2 * j] = __uint_as_float(w[i][j] << 16);
      v[i][2 * j + 1] = __uint_as_float(w[i][j] & 0xFFFF0000u);
    }
    if (c == 0 || c >= nch - 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = c * 8 + j - head;
        if (e < 0 || e >= valid) v[i][j] = -INFINITY;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, v[i][j]);
  }
  m = wave_max(m);
  const float off = 32.0f - m * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // masked elements give exp2(-inf) = 0
      v[i][j] = __builtin_amdgcn_exp2f(fmaf(v[i][j], kLog2e, off));
      sum += v[i][j];
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
      __builtin_nontemporal_store(pk, reinterpret_cast<u32x4*>(y + ay + c * 8));
    }
  }
}

template <int MAXCH>
__global__ __launch_bounds__(256) void softmax_kernel_span(
    const uint16_t* __restrict__ x, int64_t ldx, uint16_t* __restrict__ y,
    int64_t ldy, int rows, int valid, int x_bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int lane = threadIdx.x & 63;
  const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= rows) return;
  const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, x_bytes, 0x00020000);
  u32x4 w[MAXCH];
  const int64_t sx = (int64_t)row * ldx;
  if (row < rows - 1)
    softmax_span_load<MAXCH>(w, rx, sx, lane, ((int)(sx & 7) + valid + 7) >> 3);
  else
    softmax_span_load_last<MAXCH>(w, rx, x, (int64_t)row * ldx, lane, valid);
  softmax_span_row<MAXCH>(w, y, (int64_t)row * ldx, (int64_t)row * ldy, lane, valid);
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
    const float* __restrict__ mel, int C, int T, uint16_t* __restrict__ out,
    uint16_t* __restrict__ x1, int d) {
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
  // the conv1 output's pad rows (one launch less on the forward's path)
  if (x1 != nullptr && blockIdx.x == 1 % gridDim.x && blockIdx.y == 0) {
    uint16_t* xb = x1 + (int64_t)b * (T + 2) * d;
    for (int c = threadIdx.x; c < d; c += 256) {
      xb[c] = 0;
      xb[(int64_t)(T + 1) * d + c] = 0;
    }
  }
}

hipError_t launch_prep_mel(const float* mel, int batch, int C, int T,
                           uint16_t* out, hipStream_t s, uint16_t* x1, int d) {
  dim3 grid((T + 63) / 64, (C + 63) / 64, batch);
  prep_mel_kernel<<<grid, 256, 0, s>>>(mel, C, T, out, x1, d);
  return hipGetLastError();
}

}  // namespace wx
