// Kernel templates of the MFMA GEMM (gemm_dma_kernel and its epilogues,
// the register-staged fallback gemm_kernel) and their launchers, shared by
// gemm.hip (tile choice: launch_gemm, launch_gemm_i8) and the gemm_t*.hip
// translation units, each of which instantiates the launchers of a few tile
// configurations so that the library's largest compile runs in parallel.
//
// Both operands are K-contiguous (activations row-major, weights in torch's
// (out, in) layout), so every MFMA fragment is one 16-byte LDS read. The main
// kernel (gemm_dma_kernel) moves its tiles from global memory straight into
// an LDS ring with direct-to-LDS loads; the fallback (gemm_kernel, for
// operands the DMA path cannot address) stages them through registers.
// v_mfma_f32_32x32x16_bf16 operand layout (wave64):
//   A fragment: lane l holds A[row = l % 32][k = 8 * (l / 32) + 0..7]
//   B fragment: lane l holds W[col = l % 32][k = 8 * (l / 32) + 0..7]
//   C: lane l holds column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4
// The epilogue is fused: bias, GELU, residual add, the conv front end's
// padded output and positional embedding, and the QKV head split.
#pragma once

#include <utility>

#include "common.h"
#include "kernels.h"

namespace wx {

// poly4 GELU for the fc1 epilogue (g4f semantics, kernels/gelu_row4f.cc:58-84:
// the fp32 accumulator rounded to bf16 (RNE), then the RNE evaluation).
__device__ __forceinline__ float epi_poly4(float xin) {
  return poly4_gelu_pre<true>(rb_rne(xin));
}

// The GELU of a conv epilogue mode: poly4 (g4f) for the *_POLY4 modes,
// else erf.
template <int MODE>
__device__ __forceinline__ float conv_act(float x) {
  if constexpr (MODE == EPI_CONV1_POLY4 || MODE == EPI_CONV2_POLY4)
    return epi_poly4(x);
  else
    return gelu_erf(x);
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

// Write one wave's TM x TN grid of 32x32 accumulator blocks through the
// epilogue. Block (i, j) covers rows row0 + 32 i .. and columns col0 + 32 j ..;
// lane l holds column l % 32 and rows 8 g + 4 (l / 32) + r (g, r < 4). Row-
// and column-dependent parts of each output address are computed once per
// 4-row group and once per column, not per element.
template <int MODE, int TM, int TN>
__device__ __forceinline__ void store_tile(const EpiParams& e, const f32x16 (&acc)[TM][TN],
                                           int M, int N, int row0, int col0, int lane) {
  const int l32 = lane & 31, half = lane >> 5;
  int64_t cofs[TN];
  int which[TN];
  float bias[TN];
  bool cok[TN];
  static_for<TN>([&](auto j) {
    const int n = col0 + j * 32 + l32;
    cok[j] = n < N;
    const int nn = cok[j] ? n : N - 1;
    bias[j] = e.bias ? e.bias[nn] : 0.f;
    which[j] = 0;
    cofs[j] = nn;
    if (MODE == EPI_QKV) {
      const int wh = nn / e.d_model;
      const int c = nn - wh * e.d_model;
      const int h = c >> 6, dd = c & 63;
      which[j] = wh;
      cofs[j] = wh < 2 ? (int64_t)h * e.t_pad * 64 + dd
                       : (int64_t)h * 64 * e.t_pad + (int64_t)dd * e.t_pad;
    }
  });
  static_for<TM>([&](auto i) {
    static_for<4>([&](auto g) {
      const int m0 = row0 + i * 32 + g * 8 + half * 4;
      // rows m0..m0+3: batch item b and position t, one division per group
      int64_t r0[4], r1[4];
      int tt[4];
      bool rok[4];
      const int T = e.rows_per_batch;
      int b = m0 / T, t = m0 - b * T;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        rok[r] = m0 + r < M;
        tt[r] = t;
        if (MODE == EPI_CONV1)
          r0[r] = (int64_t)b * e.out_batch_stride + (int64_t)(t + 1) * e.ldo;
        else if (MODE == EPI_QKV) {
          r0[r] = ((int64_t)b * e.n_head * e.t_pad + t) * 64;
          r1[r] = (int64_t)b * e.n_head * 64 * e.t_pad + vt_key(t);
        } else
          r0[r] = (int64_t)(m0 + r) * e.ldo;
        if (++t >= T) {
          t -= T;
          ++b;
          while (t >= T) { t -= T; ++b; }
        }
      }
      static_for<TN>([&](auto j) {
        if (!cok[j]) return;
        const f32x16& a = acc[i][j];
        if (MODE == EPI_QKV && which[j] == 2) {
          // transposed V: four consecutive keys of one dim are contiguous
          const int64_t o = r1[0] + cofs[j];
          if (rok[3] && tt[3] == tt[0] + 3 && (tt[0] & 3) == 0 && (o & 3) == 0) {
            const u32x2 pk = {f2bf2(a[g * 4 + 0] + bias[j], a[g * 4 + 1] + bias[j]),
                              f2bf2(a[g * 4 + 2] + bias[j], a[g * 4 + 3] + bias[j])};
            *reinterpret_cast<u32x2*>(e.vt + o) = pk;
            return;
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!rok[r]) continue;
          float x = a[g * 4 + r] + bias[j];
          if (MODE == EPI_F32) {
            static_cast<float*>(e.out)[r0[r] + cofs[j]] = x;
          } else if (MODE == EPI_BF16) {
            if (e.gelu == GELU_ERF) x = gelu_erf(x);
            else if (e.gelu == GELU_POLY4_RNE) x = epi_poly4(x);
            static_cast<uint16_t*>(e.out)[r0[r] + cofs[j]] = f2bf(x);
          } else if (MODE == EPI_RESID) {
            float* p = static_cast<float*>(e.out) + r0[r] + cofs[j];
            *p = *p + x;
          } else if (MODE == EPI_CONV1) {
            x = e.gelu == GELU_POLY4_RNE ? epi_poly4(x) : gelu_erf(x);
            static_cast<uint16_t*>(e.out)[r0[r] + cofs[j]] = f2bf(x);
          } else if (MODE == EPI_CONV2) {
            x = e.gelu == GELU_POLY4_RNE ? epi_poly4(x) : gelu_erf(x);
            static_cast<float*>(e.out)[r0[r] + cofs[j]] = x + e.aux[(int64_t)tt[r] * N + cofs[j]];
          } else {  // EPI_QKV
            const uint16_t val = f2bf(which[j] == 0 ? x * e.q_scale : x);
            if (which[j] == 0)
              e.q[r0[r] + cofs[j]] = val;
            else if (which[j] == 1)
              e.k[r0[r] + cofs[j]] = val;
            else
              e.vt[r1[r] + cofs[j]] = val;
          }
        }
      });
    });
  });
}

// The LDS-DMA kernels multiply with the operands swapped, C^T = W . A^T, so
// that a lane's accumulator holds one ROW of C: block (i, j) covers row
// row0 + 32 i + l % 32 and columns col0 + 32 j + 8 g + 4 (l / 32) + 0..3 for
// g < 4. Each lane then writes four runs of 4 consecutive columns: 8-byte
// (bf16) or 16-byte (fp32) stores and loads, one row's address math per
// block row, and a read-modify-write of the fp32 residual in 16-byte pieces.
//
// The bias of those columns is loaded before the main loop (load_bias), so
// its latency is long gone when the epilogue runs. The activation is part of
// MODE, so each kernel carries one epilogue only. A wave tile that lies
// wholly inside C with aligned outputs (every tile but the edge ones) takes
// the unchecked path; the others check every row, column run and alignment.
template <int TN>
__device__ __forceinline__ void load_bias(const float* bias, int N, int col0, int lane,
                                          f32x4 (&bv)[TN][4]) {
  const int half = lane >> 5;
  // uniform branches only: a guarded element-wise path would make the
  // compiler wait for each load in turn, before the DMA prologue is issued
  if (bias == nullptr) {
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) { bv[j][g] = f32x4{0.f, 0.f, 0.f, 0.f}; });
    });
  } else if (((uintptr_t)bias & 15) == 0 && col0 + TN * 32 <= N) {
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) {
        bv[j][g] = *reinterpret_cast<const f32x4*>(bias + col0 + j * 32 + g * 8 + half * 4);
      });
    });
  } else {
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n0 = col0 + j * 32 + g * 8 + half * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) bv[j][g][r] = n0 + r < N ? bias[n0 + r] : 0.f;
      });
    });
  }
}

template <int MODE, int TM, int TN, bool CHECKED>
__device__ __forceinline__ void store_tile_t_impl(const EpiParams& e, const f32x16 (&acc)[TM][TN],
                                                  const f32x4 (&bv)[TN][4], int M, int N,
                                                  int row0, int col0, int lane) {
  const int l32 = lane & 31, half = lane >> 5;
  const uintptr_t ob = (uintptr_t)e.out;
  const bool v32 = !CHECKED || ((e.ldo & 3) == 0 && (ob & 15) == 0);  // fp32 runs 16-byte aligned
  const bool v16 = !CHECKED || ((e.ldo & 3) == 0 && (ob & 7) == 0);   // bf16 runs 8-byte aligned
  static_for<TM>([&](auto i) {
    const int m = row0 + i * 32 + l32;
    if (CHECKED && m >= M) return;
    int t = m;
    int64_t r0, r1 = 0;
    if (epi_conv1(MODE) || epi_conv2(MODE) || MODE == EPI_QKV) {
      const int T = e.rows_per_batch;
      const int b = m / T;
      t = m - b * T;
      if (epi_conv1(MODE)) {
        r0 = (int64_t)b * e.out_batch_stride + (int64_t)(t + 1) * e.ldo;
      } else if (MODE == EPI_QKV) {
        r0 = ((int64_t)b * e.n_head * e.t_pad + t) * 64;
        r1 = (int64_t)b * e.n_head * 64 * e.t_pad + vt_key(t);
      } else {
        r0 = (int64_t)m * e.ldo;
      }
    } else {
      r0 = (int64_t)m * e.ldo;
    }
    // The residual (EPI_RESID) or positional embedding (EPI_CONV2*) of this
    // block row is read in one batch before any of its stores: issued after
    // a store, each load would wait out a full memory round trip on its own
    // (the compiler cannot move loads above stores that may alias).
    f32x4 pre[TN][4];
    if (!CHECKED && (MODE == EPI_RESID || epi_conv2(MODE))) {
      static_for<TN>([&](auto j) {
        static_for<4>([&](auto g) {
          const int n0 = col0 + j * 32 + g * 8 + half * 4;
          pre[j][g] = MODE == EPI_RESID
                          ? *reinterpret_cast<const f32x4*>(static_cast<const float*>(e.out) + r0 + n0)
                          : *reinterpret_cast<const f32x4*>(e.aux + (int64_t)t * N + n0);
        });
      });
    }
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n0 = col0 + j * 32 + g * 8 + half * 4;
        if (CHECKED && n0 >= N) return;
        const bool full = !CHECKED || n0 + 3 < N;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = acc[i][j][g * 4 + r] + bv[j][g][r];
        if (MODE == EPI_F32 || MODE == EPI_RESID || epi_conv2(MODE)) {
          float* p = static_cast<float*>(e.out) + r0 + n0;
          if (!CHECKED) {
            f32x4 v = {x[0], x[1], x[2], x[3]};
            if (epi_conv2(MODE)) {
#pragma unroll
              for (int r = 0; r < 4; ++r) v[r] = conv_act<MODE>(v[r]) + pre[j][g][r];
            }
            if (MODE == EPI_RESID) v += pre[j][g];
            *reinterpret_cast<f32x4*>(p) = v;
            return;
          }
          if (epi_conv2(MODE)) {
            const float* ap = e.aux + (int64_t)t * N + n0;
#pragma unroll
            for (int r = 0; r < 4; ++r)
              x[r] = conv_act<MODE>(x[r]) + (full || n0 + r < N ? ap[r] : 0.f);
          }
          if (full && v32) {
            f32x4 v = {x[0], x[1], x[2], x[3]};
            if (MODE == EPI_RESID) v += *reinterpret_cast<const f32x4*>(p);
            *reinterpret_cast<f32x4*>(p) = v;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n0 + r < N) p[r] = MODE == EPI_RESID ? p[r] + x[r] : x[r];
          }
        } else if (MODE == EPI_BF16 || MODE == EPI_BF16_GELU || MODE == EPI_BF16_POLY4 ||
                   epi_conv1(MODE)) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (epi_conv1(MODE)) x[r] = conv_act<MODE>(x[r]);
            if (MODE == EPI_BF16_GELU) x[r] = gelu_erf(x[r]);
            if (MODE == EPI_BF16_POLY4) x[r] = epi_poly4(x[r]);
          }
          uint16_t* p = static_cast<uint16_t*>(e.out) + r0 + n0;
          if (full && v16) {
            const u32x2 v = {f2bf2(x[0], x[1]), f2bf2(x[2], x[3])};
            *reinterpret_cast<u32x2*>(p) = v;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n0 + r < N) p[r] = f2bf(x[r]);
          }
        } else {  // EPI_QKV: d_model % 64 == 0, so a 4-run stays in one head
          const int wh = n0 / e.d_model;
          const int c = n0 - wh * e.d_model;
          const int h = c >> 6, dd = c & 63;
          if (wh < 2) {
            uint16_t* p = (wh == 0 ? e.q : e.k) + r0 + (int64_t)h * e.t_pad * 64 + dd;
            const float sc = wh == 0 ? e.q_scale : 1.f;
            const u32x2 v = {f2bf2(x[0] * sc, x[1] * sc), f2bf2(x[2] * sc, x[3] * sc)};
            *reinterpret_cast<u32x2*>(p) = v;
          } else {
            uint16_t* p = e.vt + r1 + ((int64_t)h * 64 + dd) * e.t_pad;
#pragma unroll
            for (int r = 0; r < 4; ++r) p[(int64_t)r * e.t_pad] = f2bf(x[r]);
          }
        }
      });
    });
  });
}

template <int MODE, int TM, int TN>
__device__ __forceinline__ void store_tile_t(const EpiParams& e, const f32x16 (&acc)[TM][TN],
                                             const f32x4 (&bv)[TN][4], int M, int N, int row0,
                                             int col0, int lane) {
  const uintptr_t ob = (uintptr_t)e.out;
  const bool aligned = (e.ldo & 3) == 0 && (ob & 15) == 0;
  const bool interior = row0 + TM * 32 <= M && col0 + TN * 32 <= N &&
                        (MODE == EPI_QKV || epi_conv1(MODE) || aligned) &&
                        (!epi_conv2(MODE) || (N & 3) == 0);
  if (interior)
    store_tile_t_impl<MODE, TM, TN, false>(e, acc, bv, M, N, row0, col0, lane);
  else
    store_tile_t_impl<MODE, TM, TN, true>(e, acc, bv, M, N, row0, col0, lane);
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
    ap[i] = static_cast<const uint16_t*>(a.ptr) + (int64_t)b * a.batch_stride +
            (int64_t)t * a.lda + kc;
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

  store_tile<MODE, C::TM, C::TN>(e, acc, M, N, bm0 + wm * C::WTM, bn0 + wn * C::WTN, lane);
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

// ====================================================================
// v2: operands DMA'd straight from global memory into LDS with
// buffer_load_dwordx4 ... lds (no VGPR staging), through an S-stage ring so
// the tile S-1 K-steps ahead is already in flight while the matrix cores work
// on the current one. One such instruction writes 64 lanes x 16 bytes = 1 KB
// of LDS contiguously (lane l at byte 16*l): 1024 / (2*BK) tile rows.
// gfx950's LDS has 64 banks of 4 bytes and serves a 16-byte read for 16
// lanes per cycle, so the 16 rows those lanes read must land in 16 distinct
// 16-byte bank units. A row of 2*BK bytes covers 2*BK/256 of the banks, so an
// XOR swizzle keyed on the row bits above that puts 16-byte chunk c of row r
// in slot c ^ ((r / RPW) % CPR) (RPW rows per 256-byte bank window, CPR
// chunks per row); each DMA lane fetches the logical chunk that belongs in
// its slot. Requires K % BK == 0.
//
// DEEP = 1 (A) or 2 (W) gives that operand one slot more than the other (an
// asymmetric ring: S + 1 slots, refilled S + 1 K-steps ahead, against S),
// for the operand that streams from HBM (see launch_gemm).
template <int BM_, int BN_, int WM_, int WN_, int BK_, int STAGES_, int DEEP_ = 0>
struct DCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, S = STAGES_;
  static constexpr int DEEP = DEEP_;
  static constexpr int SA = STAGES_ + (DEEP_ == 1), SB = STAGES_ + (DEEP_ == 2);
  static constexpr int NW = WM * WN, NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int ROWB = BK * 2;            // bytes per tile row
  static constexpr int CPR = ROWB / 16;          // 16-byte chunks per row
  static constexpr int RPW = 256 / ROWB;         // rows per 256-byte bank window
  static constexpr int RPI = 1024 / ROWB;        // rows per 1 KB DMA instruction
  static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
  static constexpr int A_INSTR = A_BYTES / 1024 / NW;  // DMA instructions per wave
  static constexpr int B_INSTR = B_BYTES / 1024 / NW;
  static constexpr int IPS = A_INSTR + B_INSTR;        // per stage per wave
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int RING = SA * A_BYTES + SB * B_BYTES;  // LDS of the ring
  static_assert(BK == 32 || BK == 64 || BK == 128, "BK");
  static_assert(A_INSTR * 1024 * NW == A_BYTES && B_INSTR * 1024 * NW == B_BYTES,
                "every wave issues whole 1 KB DMA blocks");
  static_assert(TM >= 1 && TN >= 1, "wave tile");
  static_assert(S >= 2 && (S - 1) * IPS <= 63, "vmcnt immediate");
  static_assert(RING <= 160 * 1024, "LDS");
  static_assert(DEEP >= 0 && DEEP <= 2, "DEEP: 0 none, 1 A, 2 W");
};

// Tiles are walked in groups of `group_m` row-tiles (all column tiles of a
// group before the next), so concurrently running workgroups share A rows and
// W columns in L2 / the Infinity Cache. xcd_remap renumbers tile ids so that
// the ids one XCD receives (every 8th, round-robin dispatch) are a
// contiguous run of that order.
// Where the whole grid is resident at once (at most two workgroups per CU)
// and the tile grid splits evenly, `remap` kXcdBlocks instead hands XCD x
// (blockIdx % 8) block (x / pc, x % pc) of a pr x pc partition of the tile
// grid (pr = group_m, pc = 8 / pr): each XCD's L2 then holds the A rows and
// W columns of one compact block, the partition chosen for the fewest
// operand bytes per XCD.
constexpr int kGroupM = 16;
constexpr int kXcdBlocks = 2;

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4],
// lgkmcnt[11:8]; the other two counters left at their maximum, i.e. not
// waited on)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Split-K partials. A wave's accumulators (the C^T layout of store_tile_t:
// block (i, j) holds row row0 + 32 i + l % 32, columns col0 + 32 j + 8 g +
// 4 (l / 32) + 0..3) go to / come from an fp32 [M][N] slice of the
// workspace, rows and columns outside C skipped. The workgroups of one tile
// may sit on different XCDs, whose L2s are not coherent with each other:
// the partials are written and read with the sc1 cache policy (coherent at
// device scope, through to memory), so no device-wide fence -- which on
// this GPU writes back and invalidates the whole L2 -- is needed.
constexpr int kCpolSc1 = 16;

template <int TM, int TN>
__device__ __forceinline__ void sk_store(__amdgpu_buffer_rsrc_t ws, int64_t base,
                                         const f32x16 (&acc)[TM][TN], int M, int N, int row0,
                                         int col0, int lane) {
  const int l32 = lane & 31, half = lane >> 5;
  static_for<TM>([&](auto i) {
    const int m = row0 + i * 32 + l32;
    if (m >= M) return;
    const int64_t rb = base + (int64_t)m * N;
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n0 = col0 + j * 32 + g * 8 + half * 4;
        if ((N & 3) == 0 && n0 + 3 < N) {
          const f32x4 v = {acc[i][j][g * 4], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2],
                           acc[i][j][g * 4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ws,
                                                 (int)((rb + n0) * 4), 0, kCpolSc1);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n0 + r < N)
              __builtin_amdgcn_raw_buffer_store_b32(
                  __float_as_uint(acc[i][j][g * 4 + r]), ws,
                  (int)((rb + n0 + r) * 4), 0, kCpolSc1);
        }
      });
    });
  });
}

// acc <- sum over s = 0 .. splits-1 of partial s, added in that order (own
// partial `me` taken from the registers: the same values), so the result
// does not depend on which workgroup finished last.
template <int TM, int TN>
__device__ __forceinline__ void sk_reduce(__amdgpu_buffer_rsrc_t ws, int64_t slice, int splits,
                                          int me, f32x16 (&acc)[TM][TN], int M, int N,
                                          int row0, int col0, int lane) {
  const int l32 = lane & 31, half = lane >> 5;
  static_for<TM>([&](auto i) {
    const int m = row0 + i * 32 + l32;
    if (m >= M) return;
    static_for<TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n0 = col0 + j * 32 + g * 8 + half * 4;
        if (n0 >= N) return;
        const bool vec = (N & 3) == 0 && n0 + 3 < N;
        const f32x4 own = {acc[i][j][g * 4], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2],
                           acc[i][j][g * 4 + 3]};
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < splits; ++s) {
          f32x4 v = own;
          if (s != me) {
            const int64_t e0 = s * slice + (int64_t)m * N + n0;
            if (vec) {
              v = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(ws, (int)(e0 * 4), 0, kCpolSc1));
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                v[r] = n0 + r < N ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                 ws, (int)((e0 + r) * 4), 0, kCpolSc1))
                                  : 0.f;
            }
          }
          sum = s == 0 ? v : sum + v;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][g * 4 + r] = sum[r];
      });
    });
  });
}

// Epilogues through LDS, for tiles wholly inside C. In registers a lane
// holds 4-column runs of 32 different rows, so direct stores (and the fp32
// residual's loads) hand the memory pipeline 32 separate 16-byte pieces per
// instruction: ~10k cycles for a 256x256 bf16 tile and ~24k for the fp32
// residual even when every line stays in L2. Instead the finished tile is
// staged in the idle LDS ring and moved a row at a time, every memory
// instruction covering whole contiguous rows. LDS layout: row r at r * ROWB,
// 16-byte chunk q in slot q ^ (r % CPR), which keeps both the column-run
// writes and the row reads within two-way bank conflicts. Activations that
// make the epilogue VALU-bound (GELU) gain nothing here: the direct path
// already hides its stores under the arithmetic.

// (acc + bias) * mul, bf16 RNE, of the wave's tile into LDS rows
// [wm * WTM, + WTM)
template <class C>
__device__ __forceinline__ void stage_bf16(const f32x16 (&acc)[C::TM][C::TN],
                                           const f32x4 (&bv)[C::TN][4], uint8_t* smem, int wm,
                                           int wn, int lane, float mul) {
  constexpr int ROWB = C::BN * 2, CPR = ROWB / 16;
  static_assert(C::BM * ROWB <= C::RING, "staged tile fits the ring");
  const int l32 = lane & 31, half = lane >> 5;
  static_for<C::TM>([&](auto i) {
    const int r = wm * C::WTM + i * 32 + l32;
    uint8_t* rowp = smem + r * ROWB + half * 8;
    static_for<C::TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int q = (wn * C::WTN + j * 32 + g * 8) / 8;
        const f32x4 x = {(acc[i][j][g * 4] + bv[j][g][0]) * mul,
                         (acc[i][j][g * 4 + 1] + bv[j][g][1]) * mul,
                         (acc[i][j][g * 4 + 2] + bv[j][g][2]) * mul,
                         (acc[i][j][g * 4 + 3] + bv[j][g][3]) * mul};
        const u32x2 v = {f2bf2(x[0], x[1]), f2bf2(x[2], x[3])};
        *reinterpret_cast<u32x2*>(rowp + ((q ^ (r % CPR)) << 4)) = v;
      });
    });
  });
}

// plain bf16 C (EPI_BF16)
template <class C>
__device__ __forceinline__ void epi_lds_bf16(const EpiParams& e, const f32x16 (&acc)[C::TM][C::TN],
                                             const f32x4 (&bv)[C::TN][4], uint8_t* smem,
                                             int bm0, int bn0, int wm, int wn, int lane, int tid) {
  constexpr int ROWB = C::BN * 2, CPR = ROWB / 16;
  stage_bf16<C>(acc, bv, smem, wm, wn, lane, 1.f);
  __syncthreads();
  constexpr int PER = C::BM * CPR / C::NT;
  static_assert(PER * C::NT == C::BM * CPR, "whole chunks per thread");
  uint16_t* out = static_cast<uint16_t*>(e.out);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int c = tid + k * C::NT;
    const int r = c / CPR, ch = c % CPR;
    const u32x4 v = *reinterpret_cast<const u32x4*>(smem + r * ROWB + ((ch ^ (r % CPR)) << 4));
    *reinterpret_cast<u32x4*>(out + (int64_t)(bm0 + r) * e.ldo + bn0 + ch * 8) = v;
  }
}

// Q or K column tile of the fused QKV GEMM: BN / 64 whole heads; row m =
// (b, t) of head h goes to ((b * n_head + h) * t_pad + t) * 64, a 128-byte
// run per head
template <class C>
__device__ __forceinline__ void epi_lds_qk(const EpiParams& e, const f32x16 (&acc)[C::TM][C::TN],
                                           const f32x4 (&bv)[C::TN][4], uint8_t* smem, int bm0,
                                           int bn0, int wm, int wn, int lane, int tid) {
  constexpr int ROWB = C::BN * 2, CPR = ROWB / 16;
  const int wh = bn0 / e.d_model;
  stage_bf16<C>(acc, bv, smem, wm, wn, lane, wh == 0 ? e.q_scale : 1.f);
  __syncthreads();
  const int h0 = (bn0 - wh * e.d_model) >> 6;
  uint16_t* base = wh == 0 ? e.q : e.k;
  const int T = e.rows_per_batch;
  constexpr int PER = C::BM * CPR / C::NT;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int c = tid + k * C::NT;
    const int r = c / CPR, ch = c % CPR;
    const int m = bm0 + r, b = m / T, t = m - b * T;
    const u32x4 v = *reinterpret_cast<const u32x4*>(smem + r * ROWB + ((ch ^ (r % CPR)) << 4));
    *reinterpret_cast<u32x4*>(base + (((int64_t)b * e.n_head + h0 + (ch >> 3)) * e.t_pad + t) * 64 +
                              (ch & 7) * 8) = v;
  }
}

// fp32 C (EPI_F32) or C += (EPI_RESID), one wave-row band of WTM rows at a
// time (an fp32 256x256 tile is twice the ring): the band's waves stage
// acc + bias, then every thread moves whole rows, residual loads issued
// ahead of the LDS reads
template <class C, int MODE>
__device__ __forceinline__ void epi_lds_f32(const EpiParams& e, const f32x16 (&acc)[C::TM][C::TN],
                                            const f32x4 (&bv)[C::TN][4], uint8_t* smem, int bm0,
                                            int bn0, int wm, int wn, int lane, int tid) {
  constexpr int ROWB = C::BN * 4, CPR = ROWB / 16;
  static_assert(C::WTM * ROWB <= C::RING, "staged band fits the ring");
  constexpr int PER = C::WTM * CPR / C::NT;
  static_assert(PER * C::NT == C::WTM * CPR, "whole chunks per thread");
  constexpr int BATCH = PER < 8 ? PER : 8;
  static_assert(PER % BATCH == 0, "batches");
  const int l32 = lane & 31, half = lane >> 5;
  float* out = static_cast<float*>(e.out);
  static_for<C::WM>([&](auto ph) {
    if (wm == ph) {
      static_for<C::TM>([&](auto i) {
        const int r = i * 32 + l32;
        uint8_t* rowp = smem + r * ROWB;
        static_for<C::TN>([&](auto j) {
          static_for<4>([&](auto g) {
            const int q = (wn * C::WTN + j * 32 + g * 8 + half * 4) / 4;
            const f32x4 x = {acc[i][j][g * 4] + bv[j][g][0], acc[i][j][g * 4 + 1] + bv[j][g][1],
                             acc[i][j][g * 4 + 2] + bv[j][g][2],
                             acc[i][j][g * 4 + 3] + bv[j][g][3]};
            *reinterpret_cast<f32x4*>(rowp + ((q ^ (r % CPR)) << 4)) = x;
          });
        });
      });
    }
    __syncthreads();
    const int rb = bm0 + ph * C::WTM;
#pragma unroll
    for (int k0 = 0; k0 < PER; k0 += BATCH) {
      f32x4 xr[BATCH];
      if (MODE == EPI_RESID) {
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
          const int c = tid + (k0 + k) * C::NT;
          const int r = c / CPR, ch = c % CPR;
          xr[k] = *reinterpret_cast<const f32x4*>(out + (int64_t)(rb + r) * e.ldo + bn0 + ch * 4);
        }
      }
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        const int c = tid + (k0 + k) * C::NT;
        const int r = c / CPR, ch = c % CPR;
        f32x4 v = *reinterpret_cast<const f32x4*>(smem + r * ROWB + ((ch ^ (r % CPR)) << 4));
        if (MODE == EPI_RESID) v += xr[k];
        *reinterpret_cast<f32x4*>(out + (int64_t)(rb + r) * e.ldo + bn0 + ch * 4) = v;
      }
    }
    if (ph + 1 < C::WM) __syncthreads();  // the next band reuses the ring
  });
}

// I8: int8 operands (K-step of 2 BK elements: the same bytes per row as
// bf16), v_mfma_i32_32x32x32_i8 into int32 accumulators held in the same
// registers, converted and scaled (a_scale per row, w_scale per column)
// after the main loop. The v_mfma_i32_32x32x32_i8 operands are 16 bytes per
// lane like the bf16 ones, and A and W fragments are read with the same
// lane -> K mapping, so the exact integer dot product does not depend on
// how the instruction orders K inside a 32-wide slice.
template <class C, int MODE, bool I8>
__global__ __launch_bounds__(C::NT) void gemm_dma_kernel(int M, int N, int K, GemmA a,
                                                         const void* __restrict__ W,
                                                         int64_t ldw, EpiParams e,
                                                         int group_m, int remap) {
  // The buffer-resource builtins exist only for the device; the host pass
  // needs nothing but this kernel's launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::RING];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index: uniform across the wave; readfirstlane makes that visible
  // to the compiler, so everything derived from it stays in SGPRs
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / C::WN, wn = w % C::WN;
  const int l32 = lane & 31, half = lane >> 5;

  const int nm = (M + C::BM - 1) / C::BM, nn = (N + C::BN - 1) / C::BN;
  // split-K: workgroup `pid` takes split pid / tiles of tile pid % tiles,
  // i.e. K / splits of the reduction; with the XCD-contiguous order each XCD
  // then walks a compact block of tiles within one split, sharing its A rows
  // and W columns in L2
  const int splits = e.splits;
  const int ntiles = nm * nn;
  const int gid = remap ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int split = splits > 1 ? gid / ntiles : 0;
  const int tile_id = splits > 1 ? gid - split * ntiles : gid;
  const int ksplit = K / splits, kbase = split * ksplit;
  const int pid = tile_id;
  int tm, tn;
  if (remap == kXcdBlocks) {
    const int pr = group_m, pc = kXcds / pr;
    const int bmr = nm / pr, bnc = nn / pc;  // tiles per block: bmr x bnc
    const int x = blockIdx.x % kXcds, i = blockIdx.x / kXcds;
    tm = (x / pc) * bmr + i % bmr;
    tn = (x % pc) * bnc + i / bmr;
  } else {
    const int width = group_m * nn;
    const int first_m = (pid / width) * group_m;
    const int gsz = min(nm - first_m, group_m);
    tm = first_m + (pid % width) % gsz;
    tn = (pid % width) / gsz;
  }
  const int bm0 = tm * C::BM, bn0 = tn * C::BN;

  constexpr int ES = I8 ? 1 : 2;            // bytes per element
  constexpr int BKE = C::ROWB / ES;         // K elements per step

  // The buffer descriptors start at this tile's first A row and first W
  // row and cover exactly the rows the tile reads (rows past M or N are
  // clamped to the last one), so a descriptor's 32-bit extent never limits
  // the operand sizes: one tile spans at most BM rows (plus one batch
  // stride where a tile crosses a batch item of the conv windows).
  auto a_elem = [&](int m) -> int64_t {
    const int b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
    return (int64_t)b * a.batch_stride + (int64_t)t * a.lda;
  };
  const int64_t a_row0 = a_elem(bm0);
  const int64_t a_span = a_elem(min(bm0 + C::BM, M) - 1) - a_row0 + K;
  const int64_t w_span = (int64_t)(min(bn0 + C::BN, N) - 1 - bn0) * ldw + K;
  const auto ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(a.ptr)) + a_row0 * ES, (short)0,
      (int)(a_span * ES), 0x00020000);
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(W)) + (int64_t)bn0 * ldw * ES, (short)0,
      (int)(w_span * ES), 0x00020000);

  // lane -> tile row within its DMA block and the logical chunk that belongs
  // in its slot (lane % CPR) under the swizzle
  const int lrow = lane / C::CPR;
  uint32_t aoff[C::A_INSTR], boff[C::B_INSTR];
#pragma unroll
  for (int j = 0; j < C::A_INSTR; ++j) {
    const int row = (w * C::A_INSTR + j) * C::RPI + lrow;
    const int lchunk = (lane % C::CPR) ^ ((row / C::RPW) % C::CPR);
    int m = bm0 + row;
    m = m < M ? m : M - 1;
    aoff[j] = (uint32_t)((a_elem(m) - a_row0) * ES + lchunk * 16);
  }
#pragma unroll
  for (int j = 0; j < C::B_INSTR; ++j) {
    const int row = (w * C::B_INSTR + j) * C::RPI + lrow;
    const int lchunk = (lane % C::CPR) ^ ((row / C::RPW) % C::CPR);
    int n = bn0 + row;
    n = n < N ? n : N - 1;
    boff[j] = (uint32_t)((int64_t)(n - bn0) * ldw * ES + lchunk * 16);
  }
  // Asymmetric ring (DEEP): A slots [SA][A_BYTES] at the start of the ring,
  // then W slots [SB][B_BYTES]; each operand refilled on its own.
  constexpr bool ASYM = C::DEEP > 0;
  uint8_t* const wring = smem + C::SA * C::A_BYTES;
  auto issue_a = [&](int kt) {
    uint8_t* base = smem + (kt % C::SA) * C::A_BYTES;
    const int soff = (kbase + kt * BKE) * ES;
#pragma unroll
    for (int j = 0; j < C::A_INSTR; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_ptr_t)(base + (w * C::A_INSTR + j) * 1024), 16, aoff[j], soff, 0, 0);
  };
  auto issue_w = [&](int kt) {
    uint8_t* base = wring + (kt % C::SB) * C::B_BYTES;
    const int soff = (kbase + kt * BKE) * ES;
#pragma unroll
    for (int j = 0; j < C::B_INSTR; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (lds_ptr_t)(base + (w * C::B_INSTR + j) * 1024), 16, boff[j], soff, 0, 0);
  };
  auto issue = [&](int kt) {
    uint8_t* base = smem + (kt % C::S) * C::STAGE;
    const int soff = (kbase + kt * BKE) * ES;
#pragma unroll
    for (int j = 0; j < C::A_INSTR; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_ptr_t)(base + (w * C::A_INSTR + j) * 1024), 16, aoff[j], soff, 0, 0);
#pragma unroll
    for (int j = 0; j < C::B_INSTR; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (lds_ptr_t)(base + C::A_BYTES + (w * C::B_INSTR + j) * 1024), 16, boff[j],
          soff, 0, 0);
  };

  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  // issued ahead of the DMA prologue, so the first stage wait covers it too
  f32x4 bv[C::TN][4];
  load_bias<C::TN>(e.bias, N, bn0 + wn * C::WTN, lane, bv);

  const int nk = ksplit / BKE;
  const int sw = (l32 / C::RPW) % C::CPR;  // the swizzle of every row this lane reads
  const int arow = (wm * C::WTM + l32) * C::ROWB;
  const int brow = (wn * C::WTN + l32) * C::ROWB;
  constexpr int KS = C::BK / 16;  // MFMA k-slices per K-step
  constexpr int NR = C::TM + C::TN, NM = C::TM * C::TN;
  bf16x8 af[2][C::TM], bfr[2][C::TN];
  auto load_frags = [&](int stage, int kk, int set) {
    const uint8_t* As =
        ASYM ? smem + (stage % C::SA) * C::A_BYTES : smem + (stage % C::S) * C::STAGE;
    const uint8_t* Bs = ASYM ? wring + (stage % C::SB) * C::B_BYTES : As + C::A_BYTES;
    const int slot = ((kk * 2 + half) ^ sw) << 4;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
      af[set][i] = *reinterpret_cast<const bf16x8*>(As + arow + i * 32 * C::ROWB + slot);
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
      bfr[set][j] = *reinterpret_cast<const bf16x8*>(Bs + brow + j * 32 * C::ROWB + slot);
  };
  auto mfmas = [&](int set) {
    static_for<C::TM>([&](auto i) {
      static_for<C::TN>([&](auto j) {
        if constexpr (I8)
          acc[i][j] = __builtin_bit_cast(
              f32x16, __builtin_amdgcn_mfma_i32_32x32x32_i8(
                          __builtin_bit_cast(i32x4, bfr[set][j]),
                          __builtin_bit_cast(i32x4, af[set][i]),
                          __builtin_bit_cast(i32x16, acc[i][j]), 0, 0, 0));
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[set][j], af[set][i],
                                                              acc[i][j], 0, 0, 0);
      });
    });
  };

  // Pipeline. Slot (kt % S) holds K-step kt; the DMA for step kt + S is issued
  // right after the barrier of step kt, into the slot step kt just vacated.
  // Within a step, the fragments of k-slice kk+1 are read from LDS before the
  // MFMAs of slice kk are issued (each pair fenced into its own scheduling
  // region, so the reads cannot sink behind the MFMAs and share their
  // registers). The barrier, the refill and the first reads of step kt+1 sit
  // in the last slice, ahead of its MFMAs.
  // Asymmetric ring, deep operand D (S + 1 slots) and shallow H (S slots).
  // The DMA groups go out in the order D0 H0 D1 H1 .. D(S-1) H(S-1) D(S) in
  // the prologue, then H(kt+S) D(kt+S+1) after the barrier of step kt. Step
  // j's H always follows its D, so waiting for step j means waiting for
  // H(j): after it come D(j+1) and, in steady state, the S-2 whole steps
  // issued since, so D_INSTR + (S-2) IPS may stay in flight. D gets S + 1
  // steps to land, H gets S. Near the end (a refill skipped) the waits are
  // for everything.
  constexpr int D_INSTR = C::DEEP == 1 ? C::A_INSTR : C::B_INSTR;
  auto issue_d = [&](int kt) {
    if constexpr (C::DEEP == 1) issue_a(kt); else issue_w(kt);
  };
  auto issue_h = [&](int kt) {
    if constexpr (C::DEEP == 1) issue_w(kt); else issue_a(kt);
  };
  if constexpr (ASYM) {
    static_for<C::S>([&](auto i) {
      if (i < nk) {
        issue_d(i);
        issue_h(i);
      }
    });
    if (C::S < nk) issue_d(C::S);
    if (C::S < nk)
      wait_vmcnt<(C::S - 1) * C::IPS + D_INSTR>();
    else
      wait_vmcnt<0>();
  } else {
#pragma unroll
    for (int st = 0; st < C::S; ++st)
      if (st < nk) issue(st);
    if (C::S - 1 < nk)
      wait_vmcnt<(C::S - 1) * C::IPS>();
    else
      wait_vmcnt<0>();
  }
  dma_ring_barrier();
  load_frags(0, 0, 0);
  // One K-step. ISSUE: refill the slot this step frees with step kt + S;
  // NEXT: read step kt+1's first fragments. Both are compile-time, so each
  // variant is one basic block the scheduling groups below can order: after
  // the barrier the next step's first LDS reads go out first, then the DMA
  // instructions alternate one-to-one with this step's last MFMAs, so the
  // address unit drains the DMA while the matrix cores run (issued back to
  // back, the DMA would hold the wave's MFMAs behind it).
  auto step = [&](int kt, auto issue_c, auto next_c) {
    constexpr bool ISSUE = decltype(issue_c)::value, NEXT = decltype(next_c)::value;
    static_for<KS - 1>([&](auto kk) {
      load_frags(kt, kk + 1, (kk + 1) & 1);
      mfmas(kk & 1);
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);  // the reads first
      __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);  // then the MFMAs
      __builtin_amdgcn_sched_barrier(0);
    });
    // step kt+1 must have landed; issued so far are steps 0 .. kt+S-1, so the
    // S-2 steps after kt+1 may remain in flight (all of them near the end)
    if (ISSUE)
      wait_vmcnt<(C::S - 2) * C::IPS>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this step's reads done
    dma_ring_barrier();
    if (NEXT) load_frags(kt + 1, 0, 0);
    if (ISSUE) issue(kt + C::S);
    mfmas((KS - 1) & 1);
    if (NEXT) __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
    static_for<C::IPS>([&](auto) {
      if (ISSUE) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  // A step of the asymmetric ring. FULL: every refill so far and this
  // step's, H(kt+S) and D(kt+S+1), exist; otherwise each refill is issued
  // if its step exists and the wait is for everything. NEXT: read step
  // kt+1's first fragments. Same ordering of reads, MFMAs and DMA as `step`.
  auto astep = [&](int kt, auto full_c, auto next_c) {
    constexpr bool FULL = decltype(full_c)::value, NEXT = decltype(next_c)::value;
    static_for<KS - 1>([&](auto kk) {
      load_frags(kt, kk + 1, (kk + 1) & 1);
      mfmas(kk & 1);
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    if (FULL)
      wait_vmcnt<D_INSTR + (C::S - 2) * C::IPS>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this step's reads done
    dma_ring_barrier();
    if (NEXT) load_frags(kt + 1, 0, 0);
    if (FULL || kt + C::S < nk) issue_h(kt + C::S);
    if (FULL || kt + C::S + 1 < nk) issue_d(kt + C::S + 1);
    mfmas((KS - 1) & 1);
    if (NEXT) __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
    static_for<FULL ? C::IPS : 0>([&](auto) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  int kt = 0;
  if constexpr (ASYM) {
    for (; kt + C::S + 1 < nk; ++kt) astep(kt, T_{}, T_{});
    for (; kt + 1 < nk; ++kt) astep(kt, F_{}, T_{});
    if (kt < nk) astep(kt, F_{}, F_{});
  } else {
    for (; kt + C::S < nk; ++kt) step(kt, T_{}, T_{});
    for (; kt + 1 < nk; ++kt) step(kt, F_{}, T_{});
    if (kt < nk) step(kt, F_{}, F_{});
  }

  if constexpr (I8) {
    // int32 sums -> fp32 (RNE), times the row's and the column's scale, in
    // that order, each product rounded: contraction is off here, so the
    // second product cannot be fused with the epilogue's bias add into one
    // FMA (the reference rounds r * sa * sw before adding the bias; fused,
    // 6 of 7.7M fc1-shaped GELU inputs came out 1-2 ulp off). An element's
    // bits are taken with __float_as_int (a value): __builtin_bit_cast of an
    // ext-vector element lvalue reads element 0 with this compiler.
#pragma clang fp contract(off)
    const int row0 = bm0 + wm * C::WTM, col0 = bn0 + wn * C::WTN;
    float sa[C::TM];
    static_for<C::TM>([&](auto i) {
      const int m = row0 + i * 32 + l32;
      sa[i] = m < M ? e.a_scale[m] : 0.f;
    });
    const bool vec = ((uintptr_t)e.w_scale & 15) == 0 && col0 + C::TN * 32 <= N;
    static_for<C::TN>([&](auto j) {
      static_for<4>([&](auto g) {
        const int n0 = col0 + j * 32 + g * 8 + half * 4;
        f32x4 sw;
        if (vec) {
          sw = *reinterpret_cast<const f32x4*>(e.w_scale + n0);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) sw[r] = n0 + r < N ? e.w_scale[n0 + r] : 0.f;
        }
        static_for<C::TM>([&](auto i) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][g * 4 + r] =
                ((float)__float_as_int(acc[i][j][g * 4 + r]) * sa[i]) * sw[r];
        });
      });
    });
  }
  if (!I8 && splits > 1) {
    // Publish this split's partial, then count the tile's finished splits;
    // the last one sums them and runs the epilogue. No workgroup waits on
    // another, so any dispatch order completes. The flag lives in the ring's
    // first word: every LDS read and DMA of the main loop has completed
    // before its last barrier.
    int& sk_last = *reinterpret_cast<int*>(smem);
    const int64_t slice = (int64_t)M * N;
    const auto wsr = __builtin_amdgcn_make_buffer_rsrc(
        e.sk_ws, (short)0, (int)(e.sk_ws_elems * 4), 0x00020000);
    sk_store<C::TM, C::TN>(wsr, split * slice, acc, M, N, bm0 + wm * C::WTM,
                           bn0 + wn * C::WTN, lane);
    wait_vmcnt<0>();  // this thread's partial has reached the coherence point
    __syncthreads();
    if (tid == 0)
      sk_last = __hip_atomic_fetch_add(e.sk_cnt + tile_id, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(splits - 1);
    __syncthreads();
    const bool last = sk_last;
    __syncthreads();  // every wave has read the flag before the epilogue reuses LDS
    if (!last) return;
    sk_reduce<C::TM, C::TN>(wsr, slice, splits, split, acc, M, N, bm0 + wm * C::WTM,
                            bn0 + wn * C::WTN, lane);
    if (tid == 0)  // ready for the next launch
      __hip_atomic_store(e.sk_cnt + tile_id, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // EPI_F32_GELU: bias and GELU applied to the accumulators in place, then
  // the plain fp32 epilogue with a zero bias (GELU inside the staged
  // epilogue's unrolled loop would hold its temporaries next to every
  // accumulator and spill)
  constexpr int EMODE = MODE == EPI_F32_GELU ? EPI_F32 : MODE;
  if constexpr (MODE == EPI_F32_GELU) {
    static_for<C::TN>([&](auto j) {
      static_for<4>([&](auto g) {
        static_for<C::TM>([&](auto i) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][g * 4 + r] = gelu_erf(acc[i][j][g * 4 + r] + bv[j][g][r]);
        });
        bv[j][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      });
    });
  }
  // Staged epilogues (conditions uniform over the workgroup; the ring is
  // idle once every wave is past the main loop's last barrier: DMA drained,
  // fragment reads done). Their row swizzle needs a power-of-two number of
  // 16-byte chunks per row, i.e. BN a power of two; other tiles store
  // directly.
  constexpr bool kStaged = (C::BN & (C::BN - 1)) == 0;
  if (kStaged && bm0 + C::BM <= M && bn0 + C::BN <= N) {
    if constexpr (kStaged && EMODE == EPI_BF16) {
      if ((e.ldo & 7) == 0 && ((uintptr_t)e.out & 15) == 0) {
        epi_lds_bf16<C>(e, acc, bv, smem, bm0, bn0, wm, wn, lane, tid);
        return;
      }
    }
    if constexpr (kStaged && EMODE == EPI_QKV) {
      if (bn0 < 2 * e.d_model && e.d_model % C::BN == 0) {
        epi_lds_qk<C>(e, acc, bv, smem, bm0, bn0, wm, wn, lane, tid);
        return;
      }
    }
    if constexpr (kStaged && (EMODE == EPI_F32 || EMODE == EPI_RESID)) {
      if ((e.ldo & 3) == 0 && ((uintptr_t)e.out & 15) == 0) {
        epi_lds_f32<C, EMODE>(e, acc, bv, smem, bm0, bn0, wm, wn, lane, tid);
        return;
      }
    }
  }
  store_tile_t<EMODE, C::TM, C::TN>(e, acc, bv, M, N, bm0 + wm * C::WTM, bn0 + wn * C::WTN,
                                    lane);
#endif
}

template <class C, bool I8 = false>
hipError_t gemm_dma_launch(int M, int N, int K, const GemmA& a, const void* W, int64_t ldw,
                           int mode, const EpiParams& e, hipStream_t s) {
  const int tiles = ((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
  dim3 grid(tiles * e.splits), block(C::NT);
  // Tile order. Workgroups go to the 8 XCDs round-robin by id; with
  // `remap` each XCD instead walks its own contiguous run of the grouped
  // order, so the tiles one XCD runs at a time form a compact block (8 row
  // tiles x 8 column tiles for the 128x128 tile, two workgroups per CU) and
  // its L2 loads each A and W strip once. Measured with FETCH_SIZE on the
  // fc1 shape this halves the Infinity Cache / HBM reads (1.41 -> 0.76 GB)
  // and takes 5 % off the time. For the 256x256 tile (one workgroup per CU)
  // the same order in groups of 8 row tiles pays only where C is wide: an
  // XCD's 32 concurrent tiles then span 8 A strips x 4 W strips instead of
  // 2 x 16 (batch-16 fc1, 20 column tiles: 344 -> 322 us per launch, the
  // forward 0.5 ms faster in three same-box alternations); with 5 or 15
  // column tiles (fc2, out-proj, QKV) the plain grouped order measured as
  // good or better.
  const int nn_tiles = (N + C::BN - 1) / C::BN;
  const bool wide = C::BM == 256 && nn_tiles >= 20;
  int group_m = C::BM == 128 || wide ? 8 : kGroupM;
  int remap = C::BM == 128 || wide ? 1 : 0;
  // Block partition over the XCDs (batch 1: at most two 128-row tiles per CU
  // and no split): the partition with the fewest A rows + W rows per block.
  // Batch-1 large-v3 fc2 on 128x64 tiles: 4 x 2 blocks of 3 x 10 tiles
  // (3 A strips and 10 W strips per XCD) instead of runs of 30 tiles of the
  // grouped order (8 A strips and 4 W strips); the forward 4.50 -> 4.45 ms
  // in same-box alternations, same bits.
  if (C::BM == 128 && e.splits == 1 && tiles <= 2 * 256 && tiles % kXcds == 0) {
    const int nm_tiles = (M + C::BM - 1) / C::BM;
    int best = 0, best_rows = 0;
    for (int pr = 1; pr <= kXcds; pr *= 2) {
      const int pc = kXcds / pr;
      if (nm_tiles % pr || nn_tiles % pc) continue;
      const int rows = (nm_tiles / pr) * C::BM + (nn_tiles / pc) * C::BN;
      if (!best || rows < best_rows) best = pr, best_rows = rows;
    }
    if (best) group_m = best, remap = kXcdBlocks;
  }
#define WX_DMA(MD)                                                                   \
  case MD:                                                                           \
    gemm_dma_kernel<C, MD, I8><<<grid, block, 0, s>>>(M, N, K, a, W, ldw, e, group_m, \
                                                      remap);                        \
    break;
  if (mode == EPI_BF16 && e.gelu == GELU_ERF) mode = EPI_BF16_GELU;
  if (mode == EPI_BF16 && e.gelu == GELU_POLY4_RNE) mode = EPI_BF16_POLY4;
  if (mode == EPI_CONV1 && e.gelu == GELU_POLY4_RNE) mode = EPI_CONV1_POLY4;
  if (mode == EPI_CONV2 && e.gelu == GELU_POLY4_RNE) mode = EPI_CONV2_POLY4;
  if constexpr (I8) {
    // the int8 encoder's and the C ABI's epilogues
    switch (mode) {
      WX_DMA(EPI_F32) WX_DMA(EPI_BF16) WX_DMA(EPI_RESID) WX_DMA(EPI_CONV2) WX_DMA(EPI_QKV)
      WX_DMA(EPI_BF16_GELU) WX_DMA(EPI_F32_GELU)
      default:
        return hipErrorInvalidValue;
    }
  } else {
    switch (mode) {
      WX_DMA(EPI_F32) WX_DMA(EPI_BF16) WX_DMA(EPI_RESID) WX_DMA(EPI_CONV1)
      WX_DMA(EPI_CONV2) WX_DMA(EPI_QKV) WX_DMA(EPI_BF16_GELU) WX_DMA(EPI_BF16_POLY4)
      WX_DMA(EPI_CONV1_POLY4) WX_DMA(EPI_CONV2_POLY4)
      default:
        return hipErrorInvalidValue;
    }
  }
#undef WX_DMA
  return hipGetLastError();
}

using T128 = DCfg<128, 128, 2, 2, 64, 2>;
using T256w8 = DCfg<256, 256, 2, 4, 64, 2>;
using T256w8a3 = DCfg<256, 256, 2, 4, 64, 2, 1>;  // A three slots (160 KB of LDS)
using T128w8s3 = DCfg<128, 128, 2, 4, 64, 3>;
using T128w8s3w4 = DCfg<128, 128, 2, 4, 64, 3, 2>;  // W four slots (112 KB)
using T12864 = DCfg<128, 64, 2, 2, 128, 3>;         // 64x32 per wave, BK 128, 144 KB
using T12864s = DCfg<128, 64, 2, 2, 64, 3>;         // the same for K % 128 == 64, 72 KB
using T128x192 = DCfg<128, 192, 2, 2, 64, 3>;       // 64x96 per wave, 120 KB

// Instantiated in gemm_t256.hip, gemm_t128.hip, gemm_t128w8.hip and
// gemm_t12864.hip.
#define WX_GEMM_LAUNCH_DECL(C, I8)                                                        \
  template hipError_t gemm_dma_launch<C, I8>(int, int, int, const GemmA&, const void*, \
                                             int64_t, int, const EpiParams&, hipStream_t);
#define WX_GEMM_TILE_CONFIGS(X)                                                   \
  X(T256w8, false) X(T256w8, true) X(T256w8a3, false) X(T128, false) X(T128, true) \
  X(T128x192, false) X(T128w8s3, false) X(T128w8s3, true) X(T128w8s3w4, false)     \
  X(T12864, false) X(T12864, true) X(T12864s, false) X(T12864s, true)
#define WX_GEMM_EXTERN(C, I8) extern WX_GEMM_LAUNCH_DECL(C, I8)
WX_GEMM_TILE_CONFIGS(WX_GEMM_EXTERN)
#undef WX_GEMM_EXTERN

}  // namespace wx
