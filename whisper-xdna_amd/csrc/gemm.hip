// bf16 x bf16 -> fp32 MFMA GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T.
//
// Replaces the MLIR-AIE whole_array GEMM the reference drives through
// RawRT.matmul / mm_start / mm_finish (src/rawxrt.py:926-996) and the conv
// front end's im2col GEMMs (src/npu_whisper_encoder.py:422-454).
//
// Both operands are K-contiguous (activations row-major, weights in torch's
// (out, in) layout), so every MFMA fragment is one 16-byte LDS read. Tiles are
// staged global -> registers -> LDS with double buffering: the next K tile's
// global loads are in flight while the current tile feeds the matrix cores.
// v_mfma_f32_32x32x16_bf16 operand layout (wave64):
//   A fragment: lane l holds A[row = l % 32][k = 8 * (l / 32) + 0..7]
//   B fragment: lane l holds W[col = l % 32][k = 8 * (l / 32) + 0..7]
//   C: lane l holds column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4
// The epilogue is fused: bias, GELU, residual add, the conv front end's
// padded output and positional embedding, and the QKV head split.
#include "common.h"
#include "kernels.h"

namespace wx {

// poly4 GELU for the fc1 epilogue (g4f semantics: fp32 in, RNE). Constants
// kernels/gelu_poly4_coeffs.h:4-13; evaluation gelu_poly4_eval.inc:27-65.
__device__ __forceinline__ float epi_poly4(float xin) {
  const float kBreak[3] = {1.0f, 2.0f, 4.0f};
  const float kShift[3] = {0.5f, 1.5f, 3.0f};
  const float kScale[3] = {2.0f, 2.0f, 1.0f};
  const float kCoef[3][5] = {
      {-0.0020446777f, -0.013000488f, 0.077148438f, -0.06640625f, -0.15429688f},
      {0.0021514893f, -0.0071716309f, -0.0040283203f, 0.063964844f, -0.10009766f},
      {-0.0029296875f, 0.010681152f, -0.015869141f, 0.012023926f, -0.0040283203f},
  };
  const float x = rb_rne(xin);
  const float s = fabsf(x);
  float q = 0.f;
#pragma unroll
  for (int p = 2; p >= 0; --p) {
    const float u = rb_rne(rb_rne(s - kShift[p]) * kScale[p]);
    float acc = kCoef[p][0];
#pragma unroll
    for (int k = 1; k <= 4; ++k) acc = fmaf(rb_rne(acc), u, kCoef[p][k]);
    if (s < kBreak[p]) q = rb_rne(acc);
  }
  return fmaxf(x, 0.f) + q;
}

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDK = BK + 8;  // 16-byte pad: conflict-free b128 reads
  static constexpr int KCH = BK / 8;  // 16-byte chunks per tile row
  static constexpr int A_CH = BM * KCH / NT;
  static constexpr int B_CH = BN * KCH / NT;
  static_assert(A_CH * NT == BM * KCH && B_CH * NT == BN * KCH, "tile/threads");
  static_assert(TM >= 1 && TN >= 1, "wave tile");
  static constexpr int LDS_BYTES = 2 * (BM + BN) * LDK * 2;
};

// Store four consecutive rows m0..m0+3 of one column n.
template <int MODE>
__device__ __forceinline__ void epi_store4(const EpiParams& e, int m0, int n,
                                           const float* v, int M, int N) {
  if (n >= N) return;
  const float bias = e.bias ? e.bias[n] : 0.f;
  if (MODE == EPI_QKV) {
    const int d = e.d_model;
    const int which = n / d;
    const int nn = n - which * d;
    const int h = nn >> 6, dd = nn & 63;
    const int T = e.rows_per_batch;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + j;
      if (m >= M) break;
      const int b = m / T, t = m - b * T;
      const int64_t bh = (int64_t)b * e.n_head + h;
      const uint16_t val = f2bf(v[j] + bias);
      if (which == 0)
        e.q[(bh * e.t_pad + t) * 64 + dd] = val;
      else if (which == 1)
        e.k[(bh * e.t_pad + t) * 64 + dd] = val;
      else
        e.vt[(bh * 64 + dd) * e.t_pad + t] = val;
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + j;
    if (m >= M) break;
    float x = v[j] + bias;
    if (MODE == EPI_F32) {
      static_cast<float*>(e.out)[(int64_t)m * e.ldo + n] = x;
    } else if (MODE == EPI_BF16) {
      if (e.gelu == GELU_ERF) x = gelu_erf(x);
      else if (e.gelu == GELU_POLY4_RNE) x = epi_poly4(x);
      static_cast<uint16_t*>(e.out)[(int64_t)m * e.ldo + n] = f2bf(x);
    } else if (MODE == EPI_RESID) {
      float* r = static_cast<float*>(e.out) + (int64_t)m * e.ldo + n;
      *r = *r + x;
    } else if (MODE == EPI_CONV1) {
      const int T = e.rows_per_batch;
      const int b = m / T, t = m - b * T;
      static_cast<uint16_t*>(e.out)[(int64_t)b * e.out_batch_stride +
                                    (int64_t)(t + 1) * e.ldo + n] = f2bf(gelu_erf(x));
    } else if (MODE == EPI_CONV2) {
      const int T = e.rows_per_batch;
      const int t = m % T;
      static_cast<float*>(e.out)[(int64_t)m * e.ldo + n] =
          gelu_erf(x) + e.aux[(int64_t)t * N + n];
    }
  }
}

template <class C, int MODE>
__global__ __launch_bounds__(C::NT) void gemm_kernel(int M, int N, int K,
                                                     GemmA a,
                                                     const uint16_t* __restrict__ W,
                                                     int64_t ldw, EpiParams e) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][C::BM * C::LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][C::BN * C::LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  const int bm0 = blockIdx.y * C::BM;
  const int bn0 = blockIdx.x * C::BN;

  // per-thread global chunk assignment (fixed for the whole K loop)
  const uint16_t* ap[C::A_CH];
  int aoff[C::A_CH], akc[C::A_CH];
#pragma unroll
  for (int i = 0; i < C::A_CH; ++i) {
    const int c = tid + i * C::NT;
    const int r = c / C::KCH, kc = (c % C::KCH) * 8;
    int m = bm0 + r;
    m = m < M ? m : M - 1;
    const int b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
    ap[i] = a.ptr + (int64_t)b * a.batch_stride + (int64_t)t * a.lda + kc;
    aoff[i] = r * C::LDK + kc;
    akc[i] = kc;
  }
  const uint16_t* bp[C::B_CH];
  int boff[C::B_CH], bkc[C::B_CH];
#pragma unroll
  for (int i = 0; i < C::B_CH; ++i) {
    const int c = tid + i * C::NT;
    const int r = c / C::KCH, kc = (c % C::KCH) * 8;
    int n = bn0 + r;
    n = n < N ? n : N - 1;
    bp[i] = W + (int64_t)n * ldw + kc;
    boff[i] = r * C::LDK + kc;
    bkc[i] = kc;
  }

  u32x4 ra[C::A_CH], rbv[C::B_CH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i) {
      if (k0 + akc[i] < K)
        ra[i] = *reinterpret_cast<const u32x4*>(ap[i] + k0);
      else
        ra[i] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < C::B_CH; ++i) {
      if (k0 + bkc[i] < K)
        rbv[i] = *reinterpret_cast<const u32x4*>(bp[i] + k0);
      else
        rbv[i] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i)
      *reinterpret_cast<u32x4*>(&As[buf][aoff[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < C::B_CH; ++i)
      *reinterpret_cast<u32x4*>(&Bs[buf][boff[i]]) = rbv[i];
  };

  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (K + C::BK - 1) / C::BK;
  gload(0);
  sstore(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * C::BK);
#pragma unroll
    for (int kk = 0; kk < C::BK / 16; ++kk) {
      bf16x8 af[C::TM], bfr[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(
            &As[cur][(wm * C::WTM + i * 32 + frag_row) * C::LDK + kk * 16 + frag_k]);
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(
            &Bs[cur][(wn * C::WTN + j * 32 + frag_row) * C::LDK + kk * 16 + frag_k]);
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j],
                                                              acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: C fragment rows 8*g + 4*(lane/32) + (0..3), column lane % 32
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int n = bn0 + wn * C::WTN + j * 32 + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m0 = bm0 + wm * C::WTM + i * 32 + g * 8 + (lane >> 5) * 4;
        float v[4] = {acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1],
                      acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
        epi_store4<MODE>(e, m0, n, v, M, N);
      }
    }
}

template <class C>
static hipError_t gemm_launch_cfg(int M, int N, int K, const GemmA& a,
                                  const uint16_t* W, int64_t ldw, int mode,
                                  const EpiParams& e, hipStream_t s) {
  dim3 grid((N + C::BN - 1) / C::BN, (M + C::BM - 1) / C::BM);
  dim3 block(C::NT);
  switch (mode) {
    case EPI_F32:
      gemm_kernel<C, EPI_F32><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    case EPI_BF16:
      gemm_kernel<C, EPI_BF16><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    case EPI_RESID:
      gemm_kernel<C, EPI_RESID><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    case EPI_CONV1:
      gemm_kernel<C, EPI_CONV1><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    case EPI_CONV2:
      gemm_kernel<C, EPI_CONV2><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    case EPI_QKV:
      gemm_kernel<C, EPI_QKV><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

using Cfg128 = Cfg<128, 128, 64, 2, 2>;

hipError_t launch_gemm(int M, int N, int K, const GemmA& a, const uint16_t* W,
                       int64_t ldw, int mode, const EpiParams& e,
                       hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  return gemm_launch_cfg<Cfg128>(M, N, K, a, W, ldw, mode, e, s);
}

}  // namespace wx
