// Internal launch interface between the kernel files and the C-ABI / encoder.
// Every function validates nothing: callers (capi.cpp, encoder.cpp) check
// shapes, alignment and pointers first, so a launch here always fits the
// kernel's assumptions.
#pragma once

#include <hip/hip_runtime.h>

#include <vector>
#include <stdint.h>

namespace wx {

enum DType { DT_BF16 = 0, DT_F32 = 1, DT_I8 = 2 };
enum Gelu { GELU_NONE = -1, GELU_ERF = 0, GELU_POLY4_RNE = 1, GELU_POLY4_TRUNC = 2 };

// ---------------------------------------------------------------- row ops
// y = LN(x [+ resid]) * gamma + beta over each row of `cols` elements.
// sum_out (fp32, optional) receives x + resid before normalisation.
// stream: non-temporal loads and stores (for rows nothing reads again soon);
// without it, an fp32 x of 64 MB or more (no resid) still gets non-temporal
// loads, the output cached stores.
// y_dtype DT_I8: y is the row quantised per row (launch_quantize_rows'
// rule, on the fp32 LN output) with its scale in y_scale[row].
hipError_t launch_layernorm(const void* x, int x_dtype, int64_t ldx,
                            const float* resid, int64_t ldr, float* sum_out,
                            int64_t lds, const float* gamma, const float* beta,
                            float eps, void* y, int y_dtype, int64_t ldy,
                            int rows, int cols, bool stream, hipStream_t s,
                            float* y_scale = nullptr);

// Max row width the one-wave-per-row LayerNorm and softmax keep in registers.
constexpr int kMaxRowCols = 4096;

// Device tables the row kernels read (the poly4 GELU's q by bit pattern),
// written on `s`; run once per device before the first row-kernel launch.
hipError_t init_rowop_tables(hipStream_t s);

// Element-wise GELU over a rows x cols band; y is bf16.
hipError_t launch_gelu(const void* x, int x_dtype, int64_t ldx, uint16_t* y,
                       int64_t ldy, int rows, int cols, int variant,
                       hipStream_t s);

// Row softmax over the first `valid` columns of bf16 rows (fp32 internals).
hipError_t launch_softmax(const uint16_t* x, int64_t ldx, uint16_t* y,
                          int64_t ldy, int rows, int valid, hipStream_t s);

// fp32 [rows, cols] (ld ldx) -> bf16 RNE; transpose writes y[c*ldy + r].
hipError_t launch_convert(const float* x, int64_t ldx, uint16_t* y,
                          int64_t ldy, int rows, int cols, bool transpose,
                          hipStream_t s);

// ---------------------------------------------------------------- GEMM
// C[M,N] = A[M,K] . W[N,K]^T with an epilogue. A row m lives at
//   A + (m / a_rows_per_batch) * a_batch_stride + (m % a_rows_per_batch) * lda
// which covers plain row-major A (a_rows_per_batch = M) and the conv
// front-end's overlapping windows (lda = stride * channels).
enum EpiMode {
  EPI_F32 = 0,     // out fp32 = acc + bias
  EPI_BF16 = 1,    // out bf16 = gelu?(acc + bias)
  EPI_RESID = 2,   // resid fp32 += acc + bias
  EPI_CONV1 = 3,   // padded bf16 out row (t + 1) of batch b = gelu_erf(acc + bias)
  EPI_CONV2 = 4,   // resid fp32 = gelu_erf(acc + bias) + aux[t, n]
  EPI_QKV = 5,     // split into head-major Q, K and transposed V (bf16)
  // EPI_BF16 with the activation fixed at compile time (chosen by launch_gemm
  // from EpiParams::gelu; callers pass EPI_BF16)
  EPI_BF16_GELU = 6,   // out bf16 = gelu_erf(acc + bias)
  EPI_BF16_POLY4 = 7,  // out bf16 = poly4 GELU (g4f) of acc + bias
  EPI_F32_GELU = 8,    // out fp32 = gelu_erf(acc + bias)
  // EPI_CONV1 / EPI_CONV2 with the poly4 GELU (g4f) in place of erf, chosen
  // by launch_gemm from EpiParams::gelu == GELU_POLY4_RNE
  EPI_CONV1_POLY4 = 9,
  EPI_CONV2_POLY4 = 10,
};

constexpr bool epi_conv1(int m) { return m == EPI_CONV1 || m == EPI_CONV1_POLY4; }
constexpr bool epi_conv2(int m) { return m == EPI_CONV2 || m == EPI_CONV2_POLY4; }

struct GemmA {
  const void* ptr;  // bf16 (launch_gemm) or int8 (launch_gemm_i8) elements
  int64_t lda;
  int rows_per_batch;
  int64_t batch_stride;
};

struct EpiParams {
  void* out = nullptr;
  int64_t ldo = 0;
  const float* bias = nullptr;
  const float* aux = nullptr;      // positional embedding [T, N] (EPI_CONV2)
  int rows_per_batch = 1;          // T: rows of one batch item
  int64_t out_batch_stride = 0;    // EPI_CONV1: elements per padded batch item
  int gelu = GELU_NONE;            // EPI_BF16 activation; EPI_CONV*: erf unless POLY4_RNE
  uint16_t* q = nullptr;           // EPI_QKV destinations
  uint16_t* k = nullptr;
  uint16_t* vt = nullptr;
  int n_head = 0;
  int t_pad = 0;                   // padded key length of Q/K/Vt
  int d_model = 0;
  // EPI_QKV: the Q part is written as bf16((acc + bias) * q_scale), so the
  // attention kernel can take Q pre-multiplied by its softmax scale
  float q_scale = 1.f;
  // Split-K workspace (optional). With it, launch_gemm may split K over
  // `splits` workgroups per output tile when there are too few tiles to fill
  // the GPU: each writes its fp32 partial to sk_ws ([splits][M][N]), and the
  // last of a tile's workgroups to finish (per-tile counter in sk_cnt, which
  // must start zeroed and is left zeroed) sums the partials in split order
  // and runs the epilogue.
  float* sk_ws = nullptr;
  int64_t sk_ws_elems = 0;
  unsigned* sk_cnt = nullptr;
  int sk_cnt_len = 0;
  int force_splits = 0;            // 0: automatic; 1: never split; n: n splits where K allows
  int splits = 1;                  // set by launch_gemm
  // launch_gemm_i8: acc (int32) becomes (float(acc) * a_scale[row]) *
  // w_scale[col] before the bias and the epilogue
  const float* a_scale = nullptr;
  const float* w_scale = nullptr;
};

hipError_t launch_gemm(int M, int N, int K, const GemmA& a, const uint16_t* W,
                       int64_t ldw, int mode, const EpiParams& e,
                       hipStream_t s);

// int8 x int8 -> int32 MFMA GEMM with the same epilogues (no split-K): A
// int8 [M, K] with a per-row scale, W int8 [N, K] with a per-column scale.
// K % 128 == 0, lda, ldw and the batch stride multiples of 16 bytes, A and W
// 16-byte aligned (callers zero-pad K).
constexpr int kI8KAlign = 128;
hipError_t launch_gemm_i8(int M, int N, int K, const GemmA& a, const int8_t* W,
                          int64_t ldw, int mode, const EpiParams& e, hipStream_t s);

// ---------------------------------------------------------------- int8 quantisation
// Per-row symmetric quantisation: scale = max|x_row| / 127 (1 if the row is
// all zero), q = rint(x / scale) as int8, columns [cols, cols_pad) zero.
// given: scale[0] is supplied (one scale for every row) instead of computed.
hipError_t launch_quantize_rows(const void* x, int x_dtype, int64_t ldx, int rows, int cols,
                                int8_t* q, int64_t ldq, int cols_pad, float* scale,
                                bool given, hipStream_t s);
// out[0] = max|x| / 127 over a rows x cols band (1 if all zero)
hipError_t launch_absmax_scale(const void* x, int x_dtype, int64_t ldx, int rows, int cols,
                               float* out, unsigned* scratch, hipStream_t s);
// im2col of a conv1d (kernel 3, padding 1) over fp32 rows x [B, T_in, C],
// quantised per output row: row (b, t) is [x[s t - 1], x[s t], x[s t + 1]]
// (tap-major, rows outside [0, T_in) zero), padded with zeros to ldq.
hipError_t launch_im2col_quant(const float* x, int batch, int T_in, int C, int stride,
                               int T_out, int8_t* q, int64_t ldq, float* scale,
                               hipStream_t s);
// fp32 [B, C, T] -> fp32 [B, T, C]
hipError_t launch_transpose_f32(const float* x, int batch, int C, int T, float* y,
                                hipStream_t s);

// ---------------------------------------------------------------- attention
// Head dimension is fixed at 64 (Whisper: n_head = d_model / 64).
constexpr int kHeadDim = 64;
constexpr int kAttnKeyBlock = 64;
inline int attn_padded_len(int T) {
  return (T + kAttnKeyBlock - 1) / kAttnKeyBlock * kAttnKeyBlock;
}

// Position of key t in a row of Vt: within each group of 16 keys, the four
// groups of 4 are stored in the order 0, 2, 1, 3, so the 8 keys one lane
// half multiplies in the P.V MFMA (keys 4h..4h+3 and 8+4h..8+4h+3 of the
// group) are 16 contiguous bytes. Groups of 4 stay contiguous.
__host__ __device__ inline int vt_key(int t) {
  return (t & ~15) | (((t >> 2) & 1) << 3) | (((t >> 3) & 1) << 2) | (t & 3);
}

// Q, K: [B*nh, Tp, 64] bf16; Vt: [B*nh, 64, Tp] bf16 with keys placed by
// vt_key (Tp = padded T, pads finite). O row (b*T + t), column h*64 + j;
// bf16 or fp32 per o_dtype. With q_prescaled, Q already holds
// bf16(q * scale * log2(e)) (attn_q_scale), written so by the QKV GEMM's
// epilogue, and `scale` is not used.
// keysplit: 0 splits a workgroup's keys over two wave groups when there
// are fewer workgroups than CUs, 1 never does.
hipError_t launch_attention(const uint16_t* Q, const uint16_t* K,
                            const uint16_t* Vt, int batch, int n_head, int T,
                            float scale, void* O, int o_dtype, int64_t ldo,
                            hipStream_t s, bool q_prescaled = false, int keysplit = 0);

// The factor a pre-scaled Q carries: the softmax scale times log2(e), so
// that a score leaves the MFMA in the exp2 domain.
inline float attn_q_scale(float scale) { return scale * 1.4426950408889634f; }

// fp32 q, k, v rows [B*T, nh*64] (ld ld) -> the attention operand layouts.
hipError_t launch_pack_qkv(const float* q, const float* k, const float* v,
                           int64_t ld, int batch, int T, int n_head,
                           uint16_t* Q, uint16_t* K, uint16_t* Vt,
                           hipStream_t s);

// ---------------------------------------------------------------- encoder
// mel fp32 [B, C, T] -> bf16 [B, T + 2, C] with zero rows 0 and T + 1: the
// conv1 im2col becomes a window of 3 consecutive rows.
// whisper log-mel front end (audio.hip): `consts` from logmel_constants()
// on the device; out [batch][n_mels][n_samples / 160]; slots: device int
// scratch of kLogMelSlots per clip (the clip maxima), overwritten
constexpr int kLogMelSlots = 64;
std::vector<uint8_t> logmel_constants(int n_mels);
std::vector<float> mel_filterbank(int n_mels);
hipError_t launch_log_mel(const float* audio, int batch, int n_samples, int n_mels,
                          const uint8_t* consts, float* out, int* slots, hipStream_t s);
// The same on the device's file-scope scratch array (no allocation): set up
// once per device (that device current) by logmel_noalloc_setup, which
// resolves the array's address there and writes the 80- and 128-mel
// constants into it; then n_mels must be 80 or 128 and batch <=
// kNoAllocClips. Calls on one device share the array.
constexpr int kNoAllocClips = 256;
hipError_t logmel_noalloc_setup(int device);
hipError_t launch_log_mel_noalloc(int device, const float* audio, int batch, int n_samples,
                                  int n_mels, float* out, hipStream_t s);

// mel [B, C, T] fp32 -> out [B, T + 2, C] bf16 with zero rows 0 and T + 1;
// with x1 (the conv1 output [B, T + 2, d]) also zeroes x1's rows 0 and
// T + 1, which conv2's windows read as padding
hipError_t launch_prep_mel(const float* mel, int batch, int C, int T,
                           uint16_t* out, hipStream_t s, uint16_t* x1 = nullptr, int d = 0);

}  // namespace wx
