// bf16 x bf16 -> fp32 MFMA GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T, and
// its int8 x int8 -> int32 variant (launch_gemm_i8) with per-row and
// per-column scales: the tile choice per shape. The kernels and their
// launchers are in gemm_impl.h, instantiated per tile configuration in the
// gemm_t*.hip files.
//
// Replaces the MLIR-AIE whole_array GEMM the reference drives through
// RawRT.matmul / mm_start / mm_finish (src/rawxrt.py:926-996) and the conv
// front end's im2col GEMMs (src/npu_whisper_encoder.py:422-454); the int8
// variant computes the reference's quantised matmul
// (bench/probe_int8_decode.py:48-74) on the device.
#include "gemm_impl.h"

namespace wx {

// Whether one tile's operand rows fit a buffer descriptor (32-bit byte
// extent, measured from the tile's first row): at most `rows` rows of A,
// which may cross one batch item of the conv windows, and of W. The
// kernel takes A's row offsets as rising with the row index, which holds
// when every batch item's rows end before the next item starts.
static bool tile_extents_fit(int rows, int M, int K, const GemmA& a, int64_t ldw, int es) {
  const bool rising = a.rows_per_batch >= M ||
                      a.batch_stride >= (int64_t)(a.rows_per_batch - 1) * a.lda + K;
  if (!rising) return false;
  const int64_t a_span = (int64_t)rows * a.lda + a.batch_stride + K;
  const int64_t w_span = (int64_t)rows * ldw + K;
  return a_span * es < (1ll << 31) && w_span * es < (1ll << 31);
}

// Split count for a launch of `tiles` 128x128 tiles at one workgroup per
// CU: with fewer tiles than CUs, K is cut into the largest number of
// 64-multiple pieces that keeps tiles x splits within the 256 CUs and each
// piece at least 1536 long. Shorter pieces lose more to writing and reading
// the partials than they gain (measured at batch 1: fc2, K 5120, 2 splits
// 74 -> 47 us; out-proj, K 1280, 2 splits slower). e.force_splits (the
// context's tuning switch) overrides: 1 never splits, n splits n ways.
static int pick_splits(int M, int N, int K, int64_t tiles, const EpiParams& e) {
  if (!e.sk_ws || !e.sk_cnt || tiles > e.sk_cnt_len) return 1;
  auto fits = [&](int sp) {
    return K % (sp * 64) == 0 && (int64_t)sp * M * N <= e.sk_ws_elems;
  };
  if (e.force_splits > 0) return e.force_splits > 1 && fits(e.force_splits) ? e.force_splits : 1;
  for (int sp = 4; sp >= 2; --sp)
    if (tiles * sp <= 256 && K / sp >= 1536 && fits(sp)) return sp;
  return 1;
}


hipError_t launch_gemm(int M, int N, int K, const GemmA& a, const uint16_t* W,
                       int64_t ldw, int mode, const EpiParams& e_in,
                       hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  EpiParams e = e_in;
  e.splits = 1;
  const bool dma = K > 0 && K % 64 == 0 && a.lda % 8 == 0 && ldw % 8 == 0 &&
                   a.batch_stride % 8 == 0 && ((uintptr_t)a.ptr & 15) == 0 &&
                   ((uintptr_t)W & 15) == 0 && tile_extents_fit(256, M, K, a, ldw, 2);
  if (!dma) return gemm_launch_cfg<Cfg128>(M, N, K, a, W, ldw, mode, e, s);
  // Measured on MI355X over the encoder shapes with random operands: the
  // 8-wave 256x256 tile (128x64 per wave, 2 waves per SIMD, one workgroup per
  // CU) is fastest once there are enough tiles to fill the 256 CUs (batch 16:
  // fc1 367 us vs 399 for 128x128, QKV 269 vs 295, fc2 319 vs 370). Below
  // that (batch 1) the 128x128 tile keeps more CUs busy.
  // With a long K (batch-16 fc2: K 5120, A = GELU(fc1) 246 MB, too large
  // to stay in the 256 MB Infinity Cache, so every A stage comes from HBM)
  // A gets a third slot: three K-steps to land instead of two. fc2 285 vs
  // 306 us per launch, same bits; the short-K GEMMs (K 1280) gain nothing.
  const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
  if (big_tiles >= 256 && K >= 3072)
    return gemm_dma_launch<T256w8a3>(M, N, K, a, W, ldw, mode, e, s);
  if (big_tiles >= 256) return gemm_dma_launch<T256w8>(M, N, K, a, W, ldw, mode, e, s);
  // At most one 128x128 tile per CU (batch 1-2: fc2, out-proj, conv2), the
  // per-step time is the DMA latency: a 3-slot ring (one workgroup per CU)
  // keeps two steps in flight (batch 1: fc2 74 -> 54 us, out-proj 27 -> 24),
  // and split-K adds workgroups where K is long. With more tiles, two
  // workgroups per CU on the 2-slot ring do better (batch 1 QKV 29 vs 37 us).
  const int64_t tiles128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  // With a long K there (batch-1 fc2, K 5120) W, which streams from HBM
  // at batch 1 (the model's weights do not fit the Infinity Cache), gets a
  // fourth slot: fc2 47 -> 44 us per launch, same bits.
  if (tiles128 <= 256) {
    e.splits = pick_splits(M, N, K, tiles128, e);
    // Half the CUs or fewer: 128x64 tiles put twice the workgroups on the
    // CUs, each streaming 3/4 of the operand bytes per CU that a 128x128
    // tile does (the per-CU operand stream bounds these GEMMs). Once that
    // grid fills three quarters of the CUs it also beats a 2-way split of
    // the 128x128 tiles, whose fp32 partials cost more than the split gains
    // (batch-1 large-v3, 120 tiles: out-proj 15.1 -> 12.7 us run alone, the
    // forward 4.72 -> 4.61 ms; fc2 and conv2 unsplit: 4.45 -> 4.34 ms in
    // same-box alternations). A forced split (the tuning switch) stays.
    if (e.force_splits == 0 && tiles128 <= 128 && 2 * tiles128 >= 192) e.splits = 1;
    // The 128x64 tile takes K-steps of 128 (256-byte rows) where K allows:
    // with two steps in flight that is twice the bytes under way per CU, and
    // half the barriers, for the weights that stream from HBM at batch 1
    // (batch-1 forward 4.31 -> 4.21 ms in same-box alternations, same bits;
    // five 64-wide slots, the same bytes in flight, gave 4.27 ms)
    if (e.splits == 1 && tiles128 <= 128 && K % 128 == 0)
      return gemm_dma_launch<T12864>(M, N, K, a, W, ldw, mode, e, s);
    if (e.splits == 1 && tiles128 <= 128)
      return gemm_dma_launch<T12864s>(M, N, K, a, W, ldw, mode, e, s);
    if (K >= 4096) return gemm_dma_launch<T128w8s3w4>(M, N, K, a, W, ldw, mode, e, s);
    return gemm_dma_launch<T128w8s3>(M, N, K, a, W, ldw, mode, e, s);
  }
  // 257-512 tiles of 128x128 leave some CUs with two workgroups and the
  // rest with one; where 128x192 tiles come to at most 256 (batch-1 QKV:
  // 360 -> 240) every CU gets one (batch-1 forward 4.34 -> 4.30 ms, same
  // bits; the 192-wide tile stores its epilogue directly)
  const int64_t t192 = (int64_t)((M + 127) / 128) * ((N + 191) / 192);
  if (t192 <= 256) return gemm_dma_launch<T128x192>(M, N, K, a, W, ldw, mode, e, s);
  return gemm_dma_launch<T128>(M, N, K, a, W, ldw, mode, e, s);
}

// Same tile choice as launch_gemm (a K-step covers twice the int8 elements
// of a bf16 step, the same bytes); no split-K, whose fp32 partial sums would
// not be the exact integer sum.
hipError_t launch_gemm_i8(int M, int N, int K, const GemmA& a, const int8_t* W, int64_t ldw,
                          int mode, const EpiParams& e_in, hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  EpiParams e = e_in;
  e.splits = 1;
  if (K <= 0 || K % kI8KAlign || a.lda % 16 || ldw % 16 || a.batch_stride % 16 ||
      ((uintptr_t)a.ptr & 15) || ((uintptr_t)W & 15) || !tile_extents_fit(256, M, K, a, ldw, 1) ||
      !e.a_scale || !e.w_scale)
    return hipErrorInvalidValue;
  const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
  const int64_t tiles128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  if (big_tiles >= 256) return gemm_dma_launch<T256w8, true>(M, N, K, a, W, ldw, mode, e, s);
  // K-steps of 256 int8 elements on the 128x64 tile where K allows (int8
  // batch-1 forward 4.08 -> 4.00 ms)
  if (tiles128 <= 128 && K % 256 == 0)
    return gemm_dma_launch<T12864, true>(M, N, K, a, W, ldw, mode, e, s);
  if (tiles128 <= 128) return gemm_dma_launch<T12864s, true>(M, N, K, a, W, ldw, mode, e, s);
  if (tiles128 <= 256) return gemm_dma_launch<T128w8s3, true>(M, N, K, a, W, ldw, mode, e, s);
  return gemm_dma_launch<T128, true>(M, N, K, a, W, ldw, mode, e, s);
}

}  // namespace wx
