/*
 * wxhip.h -- C ABI of libwxhip.so, the MI355X (gfx950) Whisper-encoder hot
 * path. Drop-in boundary for the XDNA path of drakosha/whisper-xdna: each
 * entry point names the reference interface (file:line) whose behaviour it
 * takes over. The reference has no C ABI of its own on this path -- its
 * boundary is the Python RawRT/rowops/encoder surface -- so the Python package
 * `wxhip` (ctypes) sits on top of these functions and mirrors that surface.
 *
 * Conventions
 *  - Every function returns int: 0 (WXH_OK) or a WXH_ERR_* code. On error,
 *    wxh_last_error() returns a thread-local message. Nothing here aborts.
 *  - bf16 tensors are uint16_t bit patterns; fp32 tensors are float.
 *  - Pointers are DEVICE pointers unless the name says host. `stream` is a
 *    hipStream_t; NULL is HIP's default (null) stream, as everywhere in the
 *    HIP API (the context's own stream comes from wxh_get_stream). Calls are
 *    stream-ordered and asynchronous unless documented as synchronous.
 *  - One context is used by one host thread at a time (the reference RawRT is
 *    not thread-safe either; serve serialises it, npu_stt_server.py:131).
 */
#ifndef WXHIP_H
#define WXHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct wxh_ctx wxh_ctx;
typedef struct wxh_encoder wxh_encoder;

enum {
  WXH_OK = 0,
  WXH_ERR_INVALID = 1,     /* bad argument, shape or alignment */
  WXH_ERR_HIP = 2,         /* a HIP runtime call failed */
  WXH_ERR_INJECTED = 3,    /* fault injection (wxh_set_fail_inject) */
  WXH_ERR_UNSUPPORTED = 4, /* shape or variant outside what is built */
  WXH_ERR_STATE = 5,       /* e.g. encoder weights incomplete */
  WXH_ERR_TIMEOUT = 6      /* a blocking wait passed the context's deadline */
};

enum { WXH_BF16 = 0, WXH_F32 = 1, WXH_I8 = 2 };

/* GELU variants. ERF: exact erf-GELU (npu_whisper_encoder.py:284-287).
 * POLY4_RNE: poly4 with round-to-nearest-even (rowop codes g4r, and g4f when
 * the input is fp32; kernels/gelu_row4_rne.cc:44-66, gelu_row4f.cc:58-84).
 * POLY4_TRUNC: poly4 with truncation (rowop g4; kernels/gelu_row4.cc:44-61). */
enum { WXH_GELU_ERF = 0, WXH_GELU_POLY4_RNE = 1, WXH_GELU_POLY4_TRUNC = 2 };

/* GEMM epilogues */
enum {
  WXH_EPI_F32 = 0,             /* C fp32 = A.W^T + bias                      */
  WXH_EPI_BF16 = 1,            /* C bf16 = A.W^T + bias                      */
  WXH_EPI_BF16_GELU_ERF = 2,   /* C bf16 = gelu_erf(A.W^T + bias)            */
  WXH_EPI_BF16_GELU_POLY4 = 3, /* C bf16 = poly4 g4f (A.W^T + bias)          */
  WXH_EPI_RESID_F32 = 4,       /* C fp32 += A.W^T + bias (residual add)      */
  WXH_EPI_F32_GELU_ERF = 5     /* C fp32 = gelu_erf(A.W^T + bias) (int8 GEMM) */
};

/* Fault-injection bits: a masked entry point returns WXH_ERR_INJECTED before
 * touching the device. Mirrors the reference's forced-failure hooks
 * (tests/test_encoder_golden.py:141-147, serve/npu_stt_server.py:127-129). */
enum {
  WXH_FAIL_GEMM = 1u << 0,
  WXH_FAIL_ATTN = 1u << 1,
  WXH_FAIL_ROWOP = 1u << 2,
  WXH_FAIL_ENCODER = 1u << 3,
  WXH_FAIL_FRONTEND = 1u << 4
};

/* ------------------------------------------------------------------ context */

/* Library version string (static storage). */
const char* wxh_version(void);

/* Last error message of the calling thread ("" if none). */
const char* wxh_last_error(void);

/* Open device `device` and create a context with its own stream.
 * Replaces RawRT.__init__ (src/rawxrt.py:175-198: pyxrt.device(0), the
 * context/overlay bookkeeping). No per-shape compile, no context ceiling. */
int wxh_create(int device, wxh_ctx** out);

/* Release the caller's hold on a context. Encoders created on it keep it
 * alive; the context (its stream synchronised first) is freed when the last
 * of the caller and those encoders lets go, so wxh_destroy and
 * wxh_encoder_destroy may come in either order. */
int wxh_destroy(wxh_ctx* ctx);

/* Set the fault-injection mask (0 = off). */
int wxh_set_fail_inject(wxh_ctx* ctx, uint32_t mask);

/* The context's stream (a hipStream_t), e.g. to order caller work after it. */
int wxh_get_stream(wxh_ctx* ctx, void** stream);

/* Block until all work on the context's stream is done, or until the
 * context's deadline (wxh_set_timeout) passes: then WXH_ERR_TIMEOUT. Replaces
 * the reference's run waits (rawxrt.py:319-324, r.wait(RUN_TIMEOUT_MS)). */
int wxh_synchronize(wxh_ctx* ctx);

/* Deadline in milliseconds for every blocking wait the library makes on
 * this context and its encoders (wxh_synchronize, wxh_encoder_forward_host,
 * wxh_encoder_profile): the wait polls a completion event and gives up with
 * WXH_ERR_TIMEOUT once the deadline passes. 0 (the default) waits without a
 * deadline. The device work itself is not cancelled: it runs to completion,
 * and every buffer it uses stays owned by the library until it has (a
 * timed-out wxh_encoder_forward_host leaves the caller's output untouched).
 * The analogue of the reference's NPU_RUN_TIMEOUT_MS deadline, whose expiry
 * trips the normal fallback (rawxrt.py:51-53, 319-324). */
int wxh_set_timeout(wxh_ctx* ctx, int timeout_ms);

/* Tuning switches of a context, for tests and measurements (value 0 is the
 * automatic choice, the default):
 *  WXH_TUNE_GEMM_SPLITK: split count of the encoder GEMMs with fewer output
 *    tiles than CUs (1 never splits, n >= 2 splits K n ways where K allows);
 *  WXH_TUNE_ATTN_KEYSPLIT: 1 never splits a workgroup's keys over two wave
 *    groups (wxh_attention and the encoder's attention).
 * Encoders take the context's values when they are created. */
enum { WXH_TUNE_GEMM_SPLITK = 0, WXH_TUNE_ATTN_KEYSPLIT = 1 };
int wxh_set_tuning(wxh_ctx* ctx, int what, int value);

/* --------------------------------------------------------------- front end */

/* Log-mel spectrogram of 16 kHz mono audio: whisper's front end, which the
 * reference runs on the CPU through openai-whisper's log_mel_spectrogram
 * (tools/dump_ref.py:55-57, serve/npu_stt_server.py:334-336,
 * bench/probe_int8_decode.py:128). Centred frames of 400 samples every 160
 * (reflect padding at both ends, the last frame dropped), periodic Hann
 * window, power of the 201 DFT bins, Slaney mel filterbank
 * (librosa.filters.mel(16000, 400, n_mels)), log10(max(., 1e-10)) floored at
 * the clip's maximum - 8, then (x + 4) / 4.
 * audio: device fp32 [batch][n_samples], n_samples >= 400 (30 s windows are
 * 480000: whisper's pad_or_trim is the caller's, as in the reference);
 * out: device fp32 [batch][n_mels][n_samples / 160], the encoder's mel
 * input. The floor is taken per clip (the reference converts one window at a
 * time). The filterbank of each n_mels, and a small scratch for the clip
 * maxima (64 ints per clip, grown to the largest batch), are allocated on
 * first use and kept by the context, so calls on one context must not
 * overlap in time. Fail-inject bit WXH_FAIL_FRONTEND. */
int wxh_log_mel(wxh_ctx* ctx, const float* audio, int batch, int n_samples, int n_mels,
                float* out, void* stream);

/* wxh_log_mel without any device allocation, for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It has no counterpart in the reference. Same arguments,
 * kernels and results as wxh_log_mel; the clip-maximum scratch and the
 * filterbank constants live in a fixed device array the library holds on
 * each GPU (96 KiB, resolved and filled once per device by wxh_create).
 * Limits: batch <= 256 clips (WXH_ERR_INVALID beyond), n_mels 80 or 128
 * (WXH_ERR_UNSUPPORTED otherwise). Every call on one GPU shares that array
 * (the slots are re-initialised by each call): calls that overlap in time on
 * one GPU, from any context or stream, race. Fail-inject bit
 * WXH_FAIL_FRONTEND. */
int wxh_log_mel_noalloc(wxh_ctx* ctx, const float* audio, int batch, int n_samples,
                        int n_mels, float* out, void* stream);

/* Host-side: the mel filterbank wxh_log_mel applies, [n_mels][201] float32
 * into `out` (host memory), as librosa.filters.mel(16000, 400, n_mels)
 * builds it. Needs no GPU. */
int wxh_mel_filterbank(int n_mels, float* out);

/* ------------------------------------------------------------------ row ops */

/* y = LN(x [+ resid]) * gamma + beta over each of `rows` rows of `cols`.
 * Population variance, eps inside the sqrt (npu_whisper_encoder.py:278-281);
 * gamma/beta NULL = no affine, i.e. the rowop 'ln' of
 * kernels/layer_norm_gb.cc:48-86 (rowops.layer_norm, rowops.py:221-224).
 * x: bf16 or fp32 (x_dtype); resid: optional fp32 added first; sum_out:
 * optional fp32 receiving x + resid. y: bf16 or fp32 (y_dtype).
 * cols % 8 == 0, cols <= 4096; row strides in elements. */
int wxh_layernorm(wxh_ctx* ctx, const void* x, int x_dtype, int64_t ldx,
                  const float* resid, int64_t ldr, float* sum_out,
                  int64_t ld_sum, const float* gamma, const float* beta,
                  float eps, void* y, int y_dtype, int64_t ldy, int rows,
                  int cols, void* stream);

/* Element-wise GELU over a rows x cols band; x bf16 or fp32, y bf16.
 * Replaces RawRT.gelu / rowop g4, g4r, g4f (rawxrt.py:384-400, 546-565;
 * kernels/gelu_row4*.cc) and the numpy erf GELU (npu_whisper_encoder.py:
 * 284-300). The banded form (ldy > cols) is the g4f out_cols write of one fc1
 * chunk into fc2's A operand (rowops.py:80-88, rawxrt.py:487-516). */
int wxh_gelu(wxh_ctx* ctx, const void* x, int x_dtype, int64_t ldx,
             uint16_t* y, int64_t ldy, int rows, int cols, int variant,
             void* stream);

/* Row softmax over the first `valid` columns of each bf16 row; columns past
 * `valid` are neither read nor written. fp32 max/sum internally, RNE output.
 * Replaces rowop sm/s3/s4 and the windowed s3w/s4w/s4rw
 * (kernels/softmax_row4_body.inc:17-60, softmax_row3.cc:34-86,
 * rowops.py:60-73, 227-278) and RawRT.softmax_stack (rawxrt.py:569-585). */
int wxh_softmax_rows(wxh_ctx* ctx, const uint16_t* x, int64_t ldx,
                     uint16_t* y, int64_t ldy, int rows, int valid,
                     void* stream);

/* fp32 [rows, cols] -> bf16 (RNE); transpose != 0 writes y[c * ldy + r].
 * Replaces the host bf16 staging of RawRT._pad_into (rawxrt.py:352-371). */
int wxh_convert_f32_bf16(wxh_ctx* ctx, const float* x, int64_t ldx,
                         uint16_t* y, int64_t ldy, int rows, int cols,
                         int transpose, void* stream);

/* ------------------------------------------------------------------ GEMM */

/* C[M,N] = A[M,K] . W[N,K]^T (+ bias[N]) with an epilogue (WXH_EPI_*).
 * A, W bf16 row-major (W in torch's (out, in) layout); fp32 accumulation;
 * bias fp32 (optional). K % 8 == 0, lda % 8 == 0, ldw % 8 == 0, A and W
 * 16-byte aligned.
 * Replaces RawRT.matmul / mm_start / mm_finish (rawxrt.py:926-996) and the
 * bias fold of _pad_into (rawxrt.py:352-371; the bias stays fp32 here rather
 * than being rounded to bf16 as row K of B). */
int wxh_gemm_bf16(wxh_ctx* ctx, int M, int N, int K, const uint16_t* A,
                  int64_t lda, const uint16_t* W, int64_t ldw,
                  const float* bias, void* C, int64_t ldc, int epilogue,
                  void* stream);

/* ------------------------------------------------------------------ int8 */

/* Symmetric int8 quantisation of a rows x cols band of x (WXH_F32 or
 * WXH_BF16), the reference's quantised matmul's rule
 * (bench/probe_int8_decode.py:58-66): scale = max|x| / 127 (1 when all
 * zero), q = rint(x / scale) (round half to even) as int8, fp32 arithmetic.
 * per_tensor = 0: one scale per row, scale[rows] (per-token activations;
 * for a weight in (out, in) layout, per output channel, the reference's
 * "perchan" mode). per_tensor = 1: one scale for the band in scale[0]
 * (its "pertensor" mode). q rows hold cols_pad >= cols codes, the columns
 * past cols zero. cols % 8 == 0, ldx % 8 == 0, ldq % 8 == 0, cols_pad % 8
 * == 0, cols_pad <= 8192, x 16-byte and q 8-byte aligned. */
int wxh_quantize_rows(wxh_ctx* ctx, const void* x, int x_dtype, int64_t ldx,
                      int rows, int cols, int8_t* q, int64_t ldq, int cols_pad,
                      float* scale, int per_tensor, void* stream);

/* C[M,N] = ((float)(A_q . W_q^T)[m,n] * a_scale[m]) * w_scale[n] (+ bias[n])
 * with an epilogue (WXH_EPI_F32, _BF16, _BF16_GELU_ERF, _RESID_F32,
 * _F32_GELU_ERF). A_q int8 [M, K] (lda), W_q int8 [N, K] (ldw, torch's
 * (out, in) layout); the int32 dot products are exact and rounded once to
 * fp32, in the reference's order (bench/probe_int8_decode.py:67-71).
 * K % 128 == 0 (zero-pad K), lda % 16 == 0, ldw % 16 == 0, A and W 16-byte
 * aligned. Replaces the reference's q_matmul plug (probe_int8_decode.py:48-74)
 * for the projection, MLP and conv GEMMs. */
int wxh_gemm_i8(wxh_ctx* ctx, int M, int N, int K, const int8_t* A, int64_t lda,
                const float* a_scale, const int8_t* W, int64_t ldw,
                const float* w_scale, const float* bias, void* C, int64_t ldc,
                int epilogue, void* stream);

/* ------------------------------------------------------------------ attention */

/* Padded key length Tp used by the attention operand layouts (T rounded up
 * to the 64-key tile). */
int wxh_attention_padded_len(int T);

/* fp32 q, k, v rows [batch*T, n_head*64] (row stride ld) -> bf16 operand
 * layouts Q, K [batch*n_head, Tp, 64] and Vt [batch*n_head, 64, Tp]. The pad
 * rows/columns of Q, K, Vt must hold finite values (zero them once).
 * Replaces the host per-head staging of _attn_chain_dev
 * (rawxrt.py:848-866: transposes into the qbo/kbo/vbo sub-buffers). */
int wxh_pack_qkv(wxh_ctx* ctx, const float* q, const float* k, const float* v,
                 int64_t ld, int batch, int T, int n_head, uint16_t* Q,
                 uint16_t* K, uint16_t* Vt, void* stream);

/* O = softmax(scale * Q K^T) V per (batch, head), head dim 64, keys >= T
 * masked. O row b*T + t, columns h*64..h*64+63 (row stride ldo), bf16 or
 * fp32 (o_dtype). `scale` is the product of the reference's two hd^-1/4
 * factors, i.e. 1/sqrt(64) for Whisper.
 * Replaces RawRT.attn_chain/_attn_chain_dev (rawxrt.py:813-891) and
 * attn_fused (rawxrt.py:761-811; kernels/attn_mmul.cc:201-222). */
int wxh_attention(wxh_ctx* ctx, const uint16_t* Q, const uint16_t* K,
                  const uint16_t* Vt, int batch, int n_head, int T,
                  float scale, void* O, int o_dtype, int64_t ldo,
                  void* stream);

/* ------------------------------------------------------------------ encoder */

typedef struct {
  int n_mels;   /* 80 (tiny, small) or 128 (large-v3) */
  int d_model;  /* n_head * 64 */
  int n_head;
  int n_layer;
  int n_ctx;    /* positional-embedding rows (1500) */
  int mlp_gelu; /* WXH_GELU_ERF or WXH_GELU_POLY4_RNE (the g4f MLP of
                   RawRT.mlp, rawxrt.py:459-544) */
  int conv_gelu;/* GELU of both conv layers: WXH_GELU_ERF (the reference's
                   numpy gelu) or WXH_GELU_POLY4_RNE (its callers' E.gelu =
                   rt.gelu with GELU_OP g4r, bench/run_raw_encoder.py:82-83,
                   serve/npu_stt_server.py:203) */
} wxh_encoder_dims;

/* Create an encoder bound to `ctx`. Weights are device-resident bf16 for the
 * GEMM operands, fp32 for biases, LayerNorm and the positional embedding.
 * Replaces RawRT.register_weights + the weight BO cache (rawxrt.py:307-316,
 * 939-975) and the hw_context LRU (rawxrt.py:211-305): every weight is
 * uploaded once, nothing is evicted. */
int wxh_encoder_create(wxh_ctx* ctx, const wxh_encoder_dims* dims,
                       wxh_encoder** out);
/* Free an encoder (and its hold on its context). */
int wxh_encoder_destroy(wxh_encoder* enc);

/* Upload one weight from host fp32 by its whisper state-dict name, with or
 * without the "w." prefix of tools/dump_ref.py:72-76 ("conv1.weight",
 * "blocks.3.attn.query.weight", "positional_embedding", ...). shape must
 * match the model. Synchronous. */
int wxh_encoder_set_weight(wxh_encoder* enc, const char* name,
                           const float* host, const int64_t* shape, int ndim);

/* WXH_OK once every weight the forward needs has been set. */
int wxh_encoder_ready(wxh_encoder* enc);

/* Encoder forward: mel fp32 [batch, n_mels, n_frames] -> out fp32
 * [batch, ctx, d_model], ctx = (n_frames - 1) / 2 + 1 (<= n_ctx; the
 * positional embedding is sliced to ctx, npu_whisper_encoder.py:456-458).
 * Device pointers; stream-ordered. The body is captured into a hipGraph per
 * (batch, n_frames) on first use and replayed afterwards. An encoder's
 * workspace is shared by all its calls: a call on another stream than the
 * previous one first makes its stream wait for the previous call, and a
 * call that has to grow the workspace waits for it on the host.
 * Replaces encoder(W, mel, rt.matmul, rt.matmul, attn_fn=rt.attn_chain,
 * mlp_fn=rt.mlp) (npu_whisper_encoder.py:436-541) as driven by
 * bench/run_raw_encoder.py:79-116. */
int wxh_encoder_forward(wxh_encoder* enc, const float* mel, int batch,
                        int n_frames, float* out, void* stream);

/* Same with host buffers: copies in, runs and copies out through staging
 * buffers the encoder owns (pinned host, device; grown to the largest call),
 * synchronous under the context's deadline (wxh_set_timeout). On
 * WXH_ERR_TIMEOUT the caller's buffers are no longer in use and out_host is
 * untouched; the forward finishes on the device. */
int wxh_encoder_forward_host(wxh_encoder* enc, const float* mel_host,
                             int batch, int n_frames, float* out_host);

/* Enable (default) or disable hipGraph capture/replay of the forward body. */
int wxh_encoder_set_graph(wxh_encoder* enc, int enabled);

/* Keep int8 copies of the GEMM weights (per output channel scales, from the
 * fp32 values) as they are set; must be called before the first
 * wxh_encoder_set_weight. Needs d_model % 128 == 0 and the erf MLP GELU. */
int wxh_encoder_enable_int8(wxh_encoder* enc);

/* Run the forward with int8 GEMMs (on = 1) or bf16 (0, the default): every
 * conv, projection and MLP GEMM quantises its A operand per token and its
 * weight per output channel, as encoder(W, mel, q_matmul_factory("perchan"),
 * np_matmul, fold_bias=False) does in the reference
 * (bench/probe_int8_decode.py:48-74, 143-145); attention stays bf16 MFMA.
 * The A operands are quantised from fp32 values: the fp32 LayerNorm output
 * (in the LayerNorm kernel), the fp32 attention output, the fp32 GELU of
 * fc1, and the conv im2col rows of the fp32 mel and conv1 output. */
int wxh_encoder_set_int8(wxh_encoder* enc, int on);

/* Per-stage device time of one un-graphed forward, measured with HIP events
 * on the stream the kernels run on. ms[i] (i < n) receives the summed time
 * of stage i: 0 mel prep, 1 conv1, 2 conv2, 3 LayerNorm, 4 QKV GEMM,
 * 5 attention, 6 out-proj GEMM, 7 fc1 GEMM, 8 fc2 GEMM, 9 ln_post.
 * Synchronous. Replaces the reference's PROF/CPU_PROF stage timers
 * (rawxrt.py:69-73, npu_whisper_encoder.py:303, 409-413). */
int wxh_encoder_profile(wxh_encoder* enc, const float* mel, int batch,
                        int n_frames, float* out, float* ms, int n);

#ifdef __cplusplus
}
#endif

#endif /* WXHIP_H */
