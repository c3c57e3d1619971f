// C ABI of libwxhip.so: argument checking, error reporting, the context and
// the encoder orchestrator (device-resident weights, workspace, hipGraph).
//
// The orchestrator replaces the reference's Python-driven per-call device
// round trips (src/rawxrt.py: mm_start/mm_finish, _attn_chain_dev, _mlp_dev)
// with one stream of kernels over device-resident tensors:
//   prep_mel -> conv1 (GEMM, GELU) -> conv2 (GEMM, GELU, + pos-emb) ->
//   per layer [LN -> QKV GEMM (head split) -> attention -> out GEMM (+x) ->
//              LN -> fc1 GEMM (GELU) -> fc2 GEMM (+x)] -> ln_post
// The residual stream x stays fp32 in HBM (as the reference keeps it fp32 on
// the host, npu_whisper_encoder.py:512-527); GEMM inputs are bf16.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "../../include/wxhip.h"
#include "kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define WXH_HIP(call)                                                      \
  do {                                                                     \
    hipError_t e_ = (call);                                                \
    if (e_ != hipSuccess)                                                  \
      return fail(WXH_ERR_HIP, "%s: %s (%s:%d)", #call, hipGetErrorString(e_), \
                  __FILE__, __LINE__);                                     \
  } while (0)

#define WXH_REQUIRE(cond, ...)                          \
  do {                                                  \
    if (!(cond)) return fail(WXH_ERR_INVALID, __VA_ARGS__); \
  } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// A context is shared by its caller and by every encoder created on it; it
// is freed when the last of them lets go (wxh_destroy and
// wxh_encoder_destroy each drop one reference), so an encoder may be
// destroyed after wxh_destroy of its context, in either order.
struct wxh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t fail_mask = 0;
  std::atomic<int> refs{1};
  std::map<int, uint8_t*> logmel;  // n_mels -> device constants (log-mel front end)
  int* logmel_slots = nullptr;     // per-clip maxima scratch of wxh_log_mel
  int logmel_cap = 0;              // clips it holds
  unsigned* absmax_bits = nullptr; // per-tensor scale scratch of wxh_quantize_rows
  int timeout_ms = 0;              // deadline of the library's blocking waits (0: none)
  int tune_splitk = 0;             // WXH_TUNE_GEMM_SPLITK
  int tune_attn_keysplit = 0;      // WXH_TUNE_ATTN_KEYSPLIT
};

namespace {

// NULL is HIP's default (null) stream, exactly as in the HIP API; the
// context's own stream is available through wxh_get_stream().
hipStream_t pick(wxh_ctx*, void* s) { return static_cast<hipStream_t>(s); }

// Wait on the host until `ev` has completed, polling it, for at most
// timeout_ms (0: no deadline). The device work is never cancelled.
int wait_event(hipEvent_t ev, int timeout_ms, const char* what) {
  if (timeout_ms <= 0) {
    hipError_t e = hipEventSynchronize(ev);
    if (e != hipSuccess) return fail(WXH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return WXH_OK;
  }
  using clk = std::chrono::steady_clock;
  const auto deadline = clk::now() + std::chrono::milliseconds(timeout_ms);
  for (;;) {
    const hipError_t e = hipEventQuery(ev);
    if (e == hipSuccess) return WXH_OK;
    if (e != hipErrorNotReady)
      return fail(WXH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    if (clk::now() >= deadline)
      return fail(WXH_ERR_TIMEOUT, "%s: not complete after %d ms (the device work continues)",
                  what, timeout_ms);
    std::this_thread::sleep_for(std::chrono::microseconds(50));
  }
}

// Record an event on `s` and wait for it under the deadline.
int wait_stream(hipStream_t s, int timeout_ms, const char* what) {
  hipEvent_t ev;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return fail(WXH_ERR_HIP, "%s: hipEventCreate: %s", what, hipGetErrorString(e));
  e = hipEventRecord(ev, s);
  int r = e == hipSuccess ? wait_event(ev, timeout_ms, what)
                          : fail(WXH_ERR_HIP, "%s: hipEventRecord: %s", what, hipGetErrorString(e));
  (void)hipEventDestroy(ev);
  return r;
}

int check_ctx(wxh_ctx* c, uint32_t bit, const char* what) {
  if (!c) return fail(WXH_ERR_INVALID, "%s: null context", what);
  if (c->fail_mask & bit)
    return fail(WXH_ERR_INJECTED, "%s: injected failure (mask 0x%x)", what,
                c->fail_mask);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess)
    return fail(WXH_ERR_HIP, "%s: hipSetDevice: %s", what, hipGetErrorString(e));
  return WXH_OK;
}

}  // namespace

extern "C" {

const char* wxh_version(void) { return "wxhip 0.1 gfx950"; }

const char* wxh_last_error(void) { return g_err.c_str(); }

int wxh_create(int device, wxh_ctx** out) {
  WXH_REQUIRE(out, "wxh_create: out is null");
  int n = 0;
  WXH_HIP(hipGetDeviceCount(&n));
  WXH_REQUIRE(device >= 0 && device < n, "wxh_create: device %d of %d", device, n);
  WXH_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  WXH_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(WXH_ERR_UNSUPPORTED, "wxh_create: device %d is %s, built for gfx950",
                device, prop.gcnArchName);
  auto* c = new wxh_ctx;
  c->device = device;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return fail(WXH_ERR_HIP, "wxh_create: hipStreamCreate: %s", hipGetErrorString(e));
  }
  e = wx::init_rowop_tables(c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  // the allocation-free front end's device array: its address on this
  // device and its filterbank constants, once per device
  if (e == hipSuccess) e = wx::logmel_noalloc_setup(device);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(WXH_ERR_HIP, "wxh_create: device tables: %s", hipGetErrorString(e));
  }
  *out = c;
  return WXH_OK;
}

namespace {
void ctx_release(wxh_ctx* c) {
  if (c->refs.fetch_sub(1) != 1) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  (void)hipStreamDestroy(c->stream);
  for (auto& kv : c->logmel) (void)hipFree(kv.second);
  if (c->logmel_slots) (void)hipFree(c->logmel_slots);
  if (c->absmax_bits) (void)hipFree(c->absmax_bits);
  delete c;
}
}  // namespace

int wxh_destroy(wxh_ctx* c) {
  if (!c) return WXH_OK;
  ctx_release(c);
  return WXH_OK;
}

int wxh_set_fail_inject(wxh_ctx* c, uint32_t mask) {
  WXH_REQUIRE(c, "wxh_set_fail_inject: null context");
  c->fail_mask = mask;
  return WXH_OK;
}

int wxh_get_stream(wxh_ctx* c, void** stream) {
  WXH_REQUIRE(c && stream, "wxh_get_stream: null argument");
  *stream = c->stream;
  return WXH_OK;
}

int wxh_synchronize(wxh_ctx* c) {
  WXH_REQUIRE(c, "wxh_synchronize: null context");
  WXH_HIP(hipSetDevice(c->device));
  return wait_stream(c->stream, c->timeout_ms, "wxh_synchronize");
}

int wxh_set_timeout(wxh_ctx* c, int timeout_ms) {
  WXH_REQUIRE(c && timeout_ms >= 0, "wxh_set_timeout: null context or negative deadline");
  c->timeout_ms = timeout_ms;
  return WXH_OK;
}

int wxh_set_tuning(wxh_ctx* c, int what, int value) {
  WXH_REQUIRE(c, "wxh_set_tuning: null context");
  WXH_REQUIRE(value >= 0, "wxh_set_tuning: negative value %d", value);
  switch (what) {
    case WXH_TUNE_GEMM_SPLITK:
      WXH_REQUIRE(value <= 8, "wxh_set_tuning: split count %d > 8", value);
      c->tune_splitk = value;
      return WXH_OK;
    case WXH_TUNE_ATTN_KEYSPLIT:
      WXH_REQUIRE(value <= 1, "wxh_set_tuning: key split mode %d (0 or 1)", value);
      c->tune_attn_keysplit = value;
      return WXH_OK;
    default:
      return fail(WXH_ERR_INVALID, "wxh_set_tuning: unknown switch %d", what);
  }
}

// ------------------------------------------------------------------ row ops

int wxh_layernorm(wxh_ctx* c, const void* x, int x_dtype, int64_t ldx,
                  const float* resid, int64_t ldr, float* sum_out,
                  int64_t ld_sum, const float* gamma, const float* beta,
                  float eps, void* y, int y_dtype, int64_t ldy, int rows,
                  int cols, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ROWOP, "wxh_layernorm")) return r;
  WXH_REQUIRE(x && y, "wxh_layernorm: null x or y");
  WXH_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= wx::kMaxRowCols,
              "wxh_layernorm: cols=%d must be a positive multiple of 8 <= %d", cols,
              wx::kMaxRowCols);
  WXH_REQUIRE(x_dtype == WXH_BF16 || x_dtype == WXH_F32, "wxh_layernorm: x_dtype");
  WXH_REQUIRE(y_dtype == WXH_BF16 || y_dtype == WXH_F32, "wxh_layernorm: y_dtype");
  WXH_REQUIRE(ldx >= cols && ldy >= cols && ldx % 8 == 0 && ldy % 8 == 0,
              "wxh_layernorm: row strides must be >= cols and multiples of 8");
  WXH_REQUIRE(aligned16(x) && aligned16(y), "wxh_layernorm: x/y must be 16-byte aligned");
  WXH_REQUIRE(!resid || (ldr >= cols && ldr % 8 == 0 && aligned16(resid)),
              "wxh_layernorm: resid stride/alignment");
  WXH_REQUIRE(!sum_out || (resid && ld_sum >= cols && ld_sum % 8 == 0 && aligned16(sum_out)),
              "wxh_layernorm: sum_out needs resid and an aligned stride");
  WXH_REQUIRE(!gamma || aligned16(gamma), "wxh_layernorm: gamma alignment");
  WXH_REQUIRE(!beta || aligned16(beta), "wxh_layernorm: beta alignment");
  WXH_HIP(wx::launch_layernorm(x, x_dtype, ldx, resid, ldr, sum_out, ld_sum, gamma,
                               beta, eps, y, y_dtype, ldy, rows, cols, true,
                               pick(c, stream)));
  return WXH_OK;
}

int wxh_gelu(wxh_ctx* c, const void* x, int x_dtype, int64_t ldx, uint16_t* y,
             int64_t ldy, int rows, int cols, int variant, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ROWOP, "wxh_gelu")) return r;
  WXH_REQUIRE(x && y, "wxh_gelu: null x or y");
  WXH_REQUIRE(rows >= 0 && cols >= 0 && ldx >= cols && ldy >= cols,
              "wxh_gelu: bad shape rows=%d cols=%d ldx=%lld ldy=%lld", rows, cols,
              (long long)ldx, (long long)ldy);
  WXH_REQUIRE(x_dtype == WXH_BF16 || x_dtype == WXH_F32, "wxh_gelu: x_dtype");
  WXH_REQUIRE(variant >= WXH_GELU_ERF && variant <= WXH_GELU_POLY4_TRUNC,
              "wxh_gelu: unknown variant %d", variant);
  WXH_REQUIRE(!(variant == WXH_GELU_POLY4_TRUNC && x_dtype == WXH_F32),
              "wxh_gelu: the truncating poly4 (g4) takes bf16 input");
  WXH_HIP(wx::launch_gelu(x, x_dtype, ldx, y, ldy, rows, cols, variant, pick(c, stream)));
  return WXH_OK;
}

int wxh_softmax_rows(wxh_ctx* c, const uint16_t* x, int64_t ldx, uint16_t* y,
                     int64_t ldy, int rows, int valid, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ROWOP, "wxh_softmax_rows")) return r;
  WXH_REQUIRE(x && y, "wxh_softmax_rows: null x or y");
  WXH_REQUIRE(rows >= 0 && valid > 0 && ldx >= valid && ldy >= valid,
              "wxh_softmax_rows: bad shape rows=%d valid=%d", rows, valid);
  WXH_HIP(wx::launch_softmax(x, ldx, y, ldy, rows, valid, pick(c, stream)));
  return WXH_OK;
}

int wxh_convert_f32_bf16(wxh_ctx* c, const float* x, int64_t ldx, uint16_t* y,
                         int64_t ldy, int rows, int cols, int transpose,
                         void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ROWOP, "wxh_convert_f32_bf16")) return r;
  WXH_REQUIRE(x && y && rows >= 0 && cols >= 0 && ldx >= cols &&
                  ldy >= (transpose ? rows : cols),
              "wxh_convert_f32_bf16: bad arguments");
  WXH_HIP(wx::launch_convert(x, ldx, y, ldy, rows, cols, transpose != 0, pick(c, stream)));
  return WXH_OK;
}

// ------------------------------------------------------------- front end

int wxh_log_mel(wxh_ctx* c, const float* audio, int batch, int n_samples, int n_mels,
                float* out, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_FRONTEND, "wxh_log_mel")) return r;
  WXH_REQUIRE(audio && out, "wxh_log_mel: null pointer");
  WXH_REQUIRE(batch >= 0 && n_samples >= 400 && n_mels > 0 && n_mels <= 256,
              "wxh_log_mel: batch=%d n_samples=%d n_mels=%d", batch, n_samples, n_mels);
  auto it = c->logmel.find(n_mels);
  if (it == c->logmel.end()) {
    const std::vector<uint8_t> h = wx::logmel_constants(n_mels);
    uint8_t* d = nullptr;
    WXH_HIP(hipMalloc(&d, h.size()));
    hipError_t e = hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(d);
      return fail(WXH_ERR_HIP, "wxh_log_mel: hipMemcpy: %s", hipGetErrorString(e));
    }
    it = c->logmel.emplace(n_mels, d).first;
  }
  if (batch > c->logmel_cap) {
    if (c->logmel_slots) {
      WXH_HIP(hipDeviceSynchronize());  // an earlier call may still use it
      (void)hipFree(c->logmel_slots);
      c->logmel_slots = nullptr;
      c->logmel_cap = 0;
    }
    WXH_HIP(hipMalloc(&c->logmel_slots, (size_t)batch * wx::kLogMelSlots * sizeof(int)));
    c->logmel_cap = batch;
  }
  WXH_HIP(wx::launch_log_mel(audio, batch, n_samples, n_mels, it->second, out,
                             c->logmel_slots, pick(c, stream)));
  return WXH_OK;
}

int wxh_log_mel_noalloc(wxh_ctx* c, const float* audio, int batch, int n_samples,
                        int n_mels, float* out, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_FRONTEND, "wxh_log_mel_noalloc")) return r;
  WXH_REQUIRE(audio && out, "wxh_log_mel_noalloc: null pointer");
  WXH_REQUIRE(batch >= 0 && n_samples >= 400, "wxh_log_mel_noalloc: batch=%d n_samples=%d",
              batch, n_samples);
  WXH_REQUIRE(batch <= wx::kNoAllocClips,
              "wxh_log_mel_noalloc: batch=%d is more clips than its fixed scratch holds (%d)",
              batch, wx::kNoAllocClips);
  if (n_mels != 80 && n_mels != 128)
    return fail(WXH_ERR_UNSUPPORTED,
                "wxh_log_mel_noalloc: n_mels=%d; its fixed scratch holds the 80- and 128-mel "
                "filterbanks only (wxh_log_mel takes any)", n_mels);
  WXH_HIP(wx::launch_log_mel_noalloc(c->device, audio, batch, n_samples, n_mels, out,
                                     pick(c, stream)));
  return WXH_OK;
}

int wxh_mel_filterbank(int n_mels, float* out) {
  WXH_REQUIRE(out && n_mels > 0 && n_mels <= 256, "wxh_mel_filterbank: n_mels=%d", n_mels);
  const std::vector<float> w = wx::mel_filterbank(n_mels);
  std::memcpy(out, w.data(), w.size() * sizeof(float));
  return WXH_OK;
}

// ------------------------------------------------------------------ GEMM

int wxh_gemm_bf16(wxh_ctx* c, int M, int N, int K, const uint16_t* A,
                  int64_t lda, const uint16_t* W, int64_t ldw,
                  const float* bias, void* C, int64_t ldc, int epilogue,
                  void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_GEMM, "wxh_gemm_bf16")) return r;
  WXH_REQUIRE(A && W && C, "wxh_gemm_bf16: null operand");
  WXH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "wxh_gemm_bf16: negative size");
  WXH_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K,
              "wxh_gemm_bf16: K=%d lda=%lld ldw=%lld must be multiples of 8 (>= K)", K,
              (long long)lda, (long long)ldw);
  WXH_REQUIRE(ldc >= N, "wxh_gemm_bf16: ldc < N");
  WXH_REQUIRE(aligned16(A) && aligned16(W), "wxh_gemm_bf16: A/W must be 16-byte aligned");
  wx::EpiParams e;
  e.out = C;
  e.ldo = ldc;
  e.bias = bias;
  int mode;
  switch (epilogue) {
    case WXH_EPI_F32: mode = wx::EPI_F32; break;
    case WXH_EPI_BF16: mode = wx::EPI_BF16; break;
    case WXH_EPI_BF16_GELU_ERF: mode = wx::EPI_BF16; e.gelu = wx::GELU_ERF; break;
    case WXH_EPI_BF16_GELU_POLY4: mode = wx::EPI_BF16; e.gelu = wx::GELU_POLY4_RNE; break;
    case WXH_EPI_RESID_F32: mode = wx::EPI_RESID; break;
    default: return fail(WXH_ERR_INVALID, "wxh_gemm_bf16: unknown epilogue %d", epilogue);
  }
  wx::GemmA a{A, lda, M > 0 ? M : 1, 0};
  WXH_HIP(wx::launch_gemm(M, N, K, a, W, ldw, mode, e, pick(c, stream)));
  return WXH_OK;
}

// ------------------------------------------------------------------ int8

int wxh_quantize_rows(wxh_ctx* c, const void* x, int x_dtype, int64_t ldx, int rows,
                      int cols, int8_t* q, int64_t ldq, int cols_pad, float* scale,
                      int per_tensor, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_GEMM, "wxh_quantize_rows")) return r;
  WXH_REQUIRE(x && q && scale, "wxh_quantize_rows: null pointer");
  WXH_REQUIRE(x_dtype == WXH_F32 || x_dtype == WXH_BF16, "wxh_quantize_rows: x_dtype");
  WXH_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && ldx >= cols && ldx % 8 == 0,
              "wxh_quantize_rows: cols=%d ldx=%lld must be multiples of 8 (ldx >= cols)",
              cols, (long long)ldx);
  WXH_REQUIRE(cols_pad >= cols && cols_pad % 8 == 0 && cols_pad <= 8192 && ldq >= cols_pad &&
                  ldq % 8 == 0,
              "wxh_quantize_rows: cols_pad=%d ldq=%lld (multiples of 8, cols <= cols_pad <= "
              "8192, ldq >= cols_pad)",
              cols_pad, (long long)ldq);
  WXH_REQUIRE(aligned16(x) && ((uintptr_t)q & 7) == 0,
              "wxh_quantize_rows: x must be 16-byte and q 8-byte aligned");
  hipStream_t s = pick(c, stream);
  if (per_tensor) {
    if (!c->absmax_bits) WXH_HIP(hipMalloc(&c->absmax_bits, 256));
    WXH_HIP(wx::launch_absmax_scale(x, x_dtype, ldx, rows, cols, scale, c->absmax_bits, s));
  }
  WXH_HIP(wx::launch_quantize_rows(x, x_dtype, ldx, rows, cols, q, ldq, cols_pad, scale,
                                   per_tensor != 0, s));
  return WXH_OK;
}

int wxh_gemm_i8(wxh_ctx* c, int M, int N, int K, const int8_t* A, int64_t lda,
                const float* a_scale, const int8_t* W, int64_t ldw, const float* w_scale,
                const float* bias, void* C, int64_t ldc, int epilogue, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_GEMM, "wxh_gemm_i8")) return r;
  WXH_REQUIRE(A && W && C && a_scale && w_scale, "wxh_gemm_i8: null operand or scale");
  WXH_REQUIRE(M >= 0 && N >= 0 && K > 0, "wxh_gemm_i8: bad size");
  WXH_REQUIRE(K % wx::kI8KAlign == 0 && lda % 16 == 0 && ldw % 16 == 0 && lda >= K &&
                  ldw >= K,
              "wxh_gemm_i8: K=%d must be a multiple of %d (zero-pad), lda=%lld ldw=%lld "
              "multiples of 16 (>= K)",
              K, wx::kI8KAlign, (long long)lda, (long long)ldw);
  WXH_REQUIRE(ldc >= N, "wxh_gemm_i8: ldc < N");
  WXH_REQUIRE(aligned16(A) && aligned16(W), "wxh_gemm_i8: A/W must be 16-byte aligned");
  wx::EpiParams e;
  e.out = C;
  e.ldo = ldc;
  e.bias = bias;
  e.a_scale = a_scale;
  e.w_scale = w_scale;
  int mode;
  switch (epilogue) {
    case WXH_EPI_F32: mode = wx::EPI_F32; break;
    case WXH_EPI_BF16: mode = wx::EPI_BF16; break;
    case WXH_EPI_BF16_GELU_ERF: mode = wx::EPI_BF16; e.gelu = wx::GELU_ERF; break;
    case WXH_EPI_RESID_F32: mode = wx::EPI_RESID; break;
    case WXH_EPI_F32_GELU_ERF: mode = wx::EPI_F32_GELU; break;
    default: return fail(WXH_ERR_INVALID, "wxh_gemm_i8: unsupported epilogue %d", epilogue);
  }
  wx::GemmA a{A, lda, M > 0 ? M : 1, 0};
  WXH_HIP(wx::launch_gemm_i8(M, N, K, a, W, ldw, mode, e, pick(c, stream)));
  return WXH_OK;
}

// ------------------------------------------------------------------ attention

int wxh_attention_padded_len(int T) { return wx::attn_padded_len(T); }

int wxh_pack_qkv(wxh_ctx* c, const float* q, const float* k, const float* v,
                 int64_t ld, int batch, int T, int n_head, uint16_t* Q,
                 uint16_t* K, uint16_t* Vt, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ATTN, "wxh_pack_qkv")) return r;
  WXH_REQUIRE(q && k && v && Q && K && Vt, "wxh_pack_qkv: null pointer");
  WXH_REQUIRE(batch >= 0 && T >= 0 && n_head > 0 && ld >= (int64_t)n_head * 64,
              "wxh_pack_qkv: bad shape");
  WXH_HIP(wx::launch_pack_qkv(q, k, v, ld, batch, T, n_head, Q, K, Vt, pick(c, stream)));
  return WXH_OK;
}

int wxh_attention(wxh_ctx* c, const uint16_t* Q, const uint16_t* K,
                  const uint16_t* Vt, int batch, int n_head, int T, float scale,
                  void* O, int o_dtype, int64_t ldo, void* stream) {
  if (int r = check_ctx(c, WXH_FAIL_ATTN, "wxh_attention")) return r;
  WXH_REQUIRE(Q && K && Vt && O, "wxh_attention: null pointer");
  WXH_REQUIRE(batch >= 0 && n_head > 0 && T >= 0, "wxh_attention: bad shape");
  WXH_REQUIRE(o_dtype == WXH_BF16 || o_dtype == WXH_F32, "wxh_attention: o_dtype");
  WXH_REQUIRE(ldo >= (int64_t)n_head * 64 && ldo % 4 == 0,
              "wxh_attention: ldo must be >= n_head*64 and a multiple of 4");
  WXH_REQUIRE(aligned16(Q) && aligned16(K) && aligned16(Vt) && aligned16(O),
              "wxh_attention: operands must be 16-byte aligned");
  WXH_HIP(wx::launch_attention(Q, K, Vt, batch, n_head, T, scale, O, o_dtype, ldo,
                               pick(c, stream), false, c->tune_attn_keysplit));
  return WXH_OK;
}

}  // extern "C"

// ====================================================================== encoder

namespace {

// The encoder's LayerNorms store without the non-temporal hint: the next
// GEMM reads h straight after (with the hint on loads and stores the 64
// LayerNorms took 2.60 ms per batch-16 forward instead of 2.28).
// launch_layernorm itself puts the hint on the loads of a residual stream
// of 64 MB or more.
constexpr bool kEncLnStream = false;

struct LayerW {
  uint16_t* wqkv = nullptr;  // [3d, d]
  uint16_t* wo = nullptr;    // [d, d]
  uint16_t* w1 = nullptr;    // [ffn, d]
  uint16_t* w2 = nullptr;    // [d, ffn]
  float* bqkv = nullptr;     // [3d] (key part zero)
  float* bo = nullptr;
  float* b1 = nullptr;
  float* b2 = nullptr;
  float* ln1_g = nullptr;
  float* ln1_b = nullptr;
  float* ln2_g = nullptr;
  float* ln2_b = nullptr;
  // int8 copies (wxh_encoder_enable_int8): codes and per-output-channel scales
  int8_t* wqkv_q = nullptr;
  int8_t* wo_q = nullptr;
  int8_t* w1_q = nullptr;
  int8_t* w2_q = nullptr;
  float* sqkv = nullptr;
  float* so = nullptr;
  float* s1 = nullptr;
  float* s2 = nullptr;
};

enum Stage {
  ST_PREP = 0, ST_CONV1, ST_CONV2, ST_LN, ST_QKV, ST_ATTN, ST_OUT, ST_FC1,
  ST_FC2, ST_LNPOST, ST_COUNT
};

}  // namespace

struct wxh_encoder {
  wxh_ctx* ctx = nullptr;
  wxh_encoder_dims dims{};
  int ffn = 0;
  uint16_t* conv1_w = nullptr;  // [d, 3*n_mels], K index j*n_mels + c
  uint16_t* conv2_w = nullptr;  // [d, 3*d], K index j*d + c
  float* conv1_b = nullptr;
  float* conv2_b = nullptr;
  float* pos = nullptr;  // [n_ctx, d]
  float* lnp_g = nullptr;
  float* lnp_b = nullptr;
  std::vector<LayerW> layers;
  std::map<std::string, bool> have;
  std::vector<void*> allocs;
  // staging for fp32 uploads
  float* stage = nullptr;
  size_t stage_elems = 0;
  // workspace; capacity in elements of the largest shape seen so far
  int64_t cap_mel = 0, cap_x1 = 0, cap_x = 0, cap_qkv = 0, cap_f = 0;
  uint16_t* melT = nullptr;  // [B, T+2, n_mels]
  uint16_t* x1 = nullptr;    // [B, T+2, d]
  float* x = nullptr;        // [B*ctx, d]
  uint16_t* h = nullptr;     // [B*ctx, d]
  uint16_t* q = nullptr;     // [B*nh, Tp, 64]
  uint16_t* k = nullptr;
  uint16_t* vt = nullptr;    // [B*nh, 64, Tp]
  uint16_t* o = nullptr;     // [B*ctx, d]
  uint16_t* f = nullptr;     // [B*ctx, ffn]
  float* sk_ws = nullptr;    // split-K partials (fixed size)
  unsigned* sk_cnt = nullptr;  // split-K per-tile counters (zeroed, kept zeroed)
  std::vector<void*> ws_allocs;
  bool use_graph = true;
  std::map<std::pair<int, int>, hipGraphExec_t> graphs;
  // Calls share the workspace. `done` is recorded on a forward's stream at
  // its end: a forward on another stream first makes its stream wait for
  // it, and whatever frees or rewrites memory a forward reads (workspace
  // regrow, weights, graphs, the staging buffers, destroy) waits for it on
  // the host.
  hipEvent_t done = nullptr;
  bool done_pending = false;
  hipStream_t last_stream = nullptr;
  int tune_splitk = 0, tune_attn_keysplit = 0;  // the context's, at creation
  // wxh_encoder_forward_host staging: pinned host and device copies of the
  // mel and the features, grown to the largest call
  float* h_mel = nullptr;
  float* h_out = nullptr;
  float* d_mel = nullptr;
  float* d_out = nullptr;
  size_t cap_io_in = 0, cap_io_out = 0;
  // int8 GEMM path
  bool i8_weights = false;   // int8 weight copies are kept (enable_int8)
  bool i8 = false;           // the forward runs the int8 path (set_int8)
  int k1p = 0;               // conv1 K (3 n_mels) padded to a multiple of 128
  int8_t* conv1_q = nullptr; // [d, k1p], K index j*n_mels + c
  int8_t* conv2_q = nullptr; // [d, 3d]
  float* conv1_s = nullptr;
  float* conv2_s = nullptr;
  int64_t cap_aq = 0, cap_asc = 0, cap_f32 = 0;
  int8_t* aq = nullptr;      // quantised A operand of the current GEMM
  float* asc = nullptr;      // its per-row scales
  float* f32ws = nullptr;    // fp32 staging: mel^T, conv1 out, attention out, GELU(fc1)
};

namespace {

template <class T>
int dalloc(std::vector<void*>& list, T** p, size_t count, bool zero) {
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, count * sizeof(T) + 256);
  if (e != hipSuccess)
    return fail(WXH_ERR_HIP, "hipMalloc(%zu bytes): %s", count * sizeof(T),
                hipGetErrorString(e));
  if (zero) {
    e = hipMemset(d, 0, count * sizeof(T) + 256);
    if (e != hipSuccess) {
      (void)hipFree(d);
      return fail(WXH_ERR_HIP, "hipMemset: %s", hipGetErrorString(e));
    }
  }
  list.push_back(d);
  *p = static_cast<T*>(d);
  return WXH_OK;
}

void free_list(std::vector<void*>& list) {
  for (void* p : list) (void)hipFree(p);
  list.clear();
}

// Host wait for the encoder's last forward; bounded by the context's
// deadline unless `bounded` is false (before memory is freed).
int quiesce(wxh_encoder* E, const char* what, bool bounded = true) {
  if (!E->done_pending) return WXH_OK;
  const int r = wait_event(E->done, bounded ? E->ctx->timeout_ms : 0, what);
  if (r == WXH_OK) E->done_pending = false;
  return r;
}

void drop_graphs(wxh_encoder* E) {
  for (auto& kv : E->graphs) (void)hipGraphExecDestroy(kv.second);
  E->graphs.clear();
}

int ensure_stage(wxh_encoder* E, size_t n) {
  if (E->stage_elems >= n) return WXH_OK;
  if (E->stage) (void)hipFree(E->stage);
  E->stage = nullptr;
  E->stage_elems = 0;
  WXH_HIP(hipMalloc(&E->stage, n * sizeof(float)));
  E->stage_elems = n;
  return WXH_OK;
}

// host fp32 [rows, cols] -> device bf16 via the conversion kernel (RNE);
// with q, also int8 codes [rows, q_ld] and a scale per row (output
// channel), quantised from the fp32 values
int upload_bf16(wxh_encoder* E, uint16_t* dst, const float* host, int rows, int cols,
                int8_t* q = nullptr, float* q_scale = nullptr, int q_ld = 0) {
  const size_t n = (size_t)rows * cols;
  if (int r = ensure_stage(E, n)) return r;
  hipStream_t s = E->ctx->stream;
  WXH_HIP(hipMemcpyAsync(E->stage, host, n * sizeof(float), hipMemcpyHostToDevice, s));
  WXH_HIP(wx::launch_convert(E->stage, cols, dst, cols, rows, cols, false, s));
  if (q)
    WXH_HIP(wx::launch_quantize_rows(E->stage, wx::DT_F32, cols, rows, cols, q, q_ld, q_ld,
                                     q_scale, false, s));
  WXH_HIP(hipStreamSynchronize(s));
  return WXH_OK;
}

int upload_f32(wxh_encoder* E, float* dst, const float* host, size_t n) {
  WXH_HIP(hipMemcpy(dst, host, n * sizeof(float), hipMemcpyHostToDevice));
  return WXH_OK;
}

bool shape_is(const int64_t* shape, int ndim, std::initializer_list<int64_t> want) {
  if ((size_t)ndim != want.size()) return false;
  int i = 0;
  for (int64_t w : want)
    if (shape[i++] != w) return false;
  return true;
}

std::vector<std::string> required_names(const wxh_encoder_dims& d) {
  std::vector<std::string> v = {"conv1.weight", "conv1.bias", "conv2.weight",
                                "conv2.bias", "positional_embedding",
                                "ln_post.weight", "ln_post.bias"};
  for (int L = 0; L < d.n_layer; ++L) {
    const std::string p = "blocks." + std::to_string(L) + ".";
    for (const char* s :
         {"attn_ln.weight", "attn_ln.bias", "attn.query.weight", "attn.query.bias",
          "attn.key.weight", "attn.value.weight", "attn.value.bias", "attn.out.weight",
          "attn.out.bias", "mlp_ln.weight", "mlp_ln.bias", "mlp.0.weight", "mlp.0.bias",
          "mlp.2.weight", "mlp.2.bias"})
      v.push_back(p + s);
  }
  return v;
}

constexpr int64_t kSplitKElems = 512ll * 128 * 128;  // 32 MiB of fp32
constexpr int kSplitKTiles = 512;

int ensure_workspace(wxh_encoder* E, int batch, int frames) {
  const auto& D = E->dims;
  const int64_t B = batch, T = frames;
  const int64_t ctx = (T - 1) / 2 + 1;
  const int64_t tp = wx::attn_padded_len((int)ctx);
  const int64_t need_mel = B * (T + 2) * D.n_mels;
  const int64_t need_x1 = B * (T + 2) * D.d_model;
  const int64_t need_x = B * ctx * D.d_model;
  const int64_t need_qkv = B * D.n_head * tp * 64;
  const int64_t need_f = B * ctx * E->ffn;
  // int8 path: the quantised A operand (conv1 im2col, conv2 im2col or
  // [M, ffn]), its row scales, and fp32 staging
  const int64_t d = D.d_model;
  const int64_t need_aq =
      E->i8 ? std::max({B * T * E->k1p, B * ctx * 3 * d, B * ctx * E->ffn}) : 0;
  const int64_t need_asc = E->i8 ? B * T : 0;
  const int64_t need_f32 =
      E->i8 ? std::max({B * T * (int64_t)D.n_mels, B * T * d, B * ctx * E->ffn}) : 0;
  if (need_mel <= E->cap_mel && need_x1 <= E->cap_x1 && need_x <= E->cap_x &&
      need_qkv <= E->cap_qkv && need_f <= E->cap_f && need_aq <= E->cap_aq &&
      need_asc <= E->cap_asc && need_f32 <= E->cap_f32)
    return WXH_OK;
  if (int r = quiesce(E, "encoder workspace regrow", false)) return r;
  drop_graphs(E);
  free_list(E->ws_allocs);
  E->cap_mel = E->cap_x1 = E->cap_x = E->cap_qkv = E->cap_f = 0;
  E->cap_aq = E->cap_asc = E->cap_f32 = 0;
  auto& L = E->ws_allocs;
  // pads (conv rows, attention key/query tails) must hold finite values:
  // everything starts zeroed, and later writes only ever store finite bf16
  if (int r = dalloc(L, &E->melT, need_mel, true)) return r;
  if (int r = dalloc(L, &E->x1, need_x1, true)) return r;
  if (int r = dalloc(L, &E->x, need_x, true)) return r;
  if (int r = dalloc(L, &E->h, need_x, true)) return r;
  if (int r = dalloc(L, &E->q, need_qkv, true)) return r;
  if (int r = dalloc(L, &E->k, need_qkv, true)) return r;
  if (int r = dalloc(L, &E->vt, need_qkv, true)) return r;
  if (int r = dalloc(L, &E->o, need_x, true)) return r;
  if (int r = dalloc(L, &E->f, need_f, true)) return r;
  if (int r = dalloc(L, &E->sk_ws, (size_t)kSplitKElems, false)) return r;
  if (int r = dalloc(L, &E->sk_cnt, (size_t)kSplitKTiles, true)) return r;
  if (E->i8) {
    if (int r = dalloc(L, &E->aq, (size_t)need_aq, true)) return r;
    if (int r = dalloc(L, &E->asc, (size_t)need_asc, true)) return r;
    if (int r = dalloc(L, &E->f32ws, (size_t)need_f32, true)) return r;
    E->cap_aq = need_aq;
    E->cap_asc = need_asc;
    E->cap_f32 = need_f32;
  }
  E->cap_mel = need_mel;
  E->cap_x1 = need_x1;
  E->cap_x = need_x;
  E->cap_qkv = need_qkv;
  E->cap_f = need_f;
  return WXH_OK;
}

// Split-K for the GEMMs whose tile count leaves CUs idle (batch 1-2): one
// partial slice per split of C, at most 512 workgroups of 128x128 tiles.
void set_splitk(wxh_encoder* E, wx::EpiParams& e) {
  e.sk_ws = E->sk_ws;
  e.sk_ws_elems = kSplitKElems;
  e.sk_cnt = E->sk_cnt;
  e.sk_cnt_len = kSplitKTiles;
  e.force_splits = E->tune_splitk;
}

struct StageTimer {
  std::vector<std::pair<int, hipEvent_t>> marks;
  hipEvent_t start = nullptr;
};

// Launch the forward body (conv1 .. last layer). Stage events are recorded
// after each launch when `timer` is set (un-graphed profiling only).
// The int8 forward body. Every GEMM takes int8 A (quantised per row) and W
// (per output channel) and runs launch_gemm_i8; the A operands come from
// fp32 values: the conv im2col rows of the transposed fp32 mel (f32ws,
// written before the graph) and of the fp32 conv1 output, the LayerNorm's
// fp32 result (quantised in the LayerNorm kernel), the fp32 attention
// output and the fp32 GELU(fc1).
int run_body_i8(wxh_encoder* E, int batch, int frames, hipStream_t s, StageTimer* timer) {
  const auto& D = E->dims;
  const int d = D.d_model, nh = D.n_head, T = frames, C = D.n_mels;
  const int ctx = (T - 1) / 2 + 1;
  const int tp = wx::attn_padded_len(ctx);
  const int M = batch * ctx, ffn = E->ffn;
  auto mark = [&](int stage) -> int {
    if (!timer) return WXH_OK;
    hipEvent_t ev;
    WXH_HIP(hipEventCreate(&ev));
    WXH_HIP(hipEventRecord(ev, s));
    timer->marks.push_back({stage, ev});
    return WXH_OK;
  };
  auto gemm = [&](int m, int n, int k, const int8_t* w, const float* wsc, int mode,
                  wx::EpiParams e) -> int {
    e.a_scale = E->asc;
    e.w_scale = wsc;
    wx::GemmA a{E->aq, k, m, 0};
    WXH_HIP(wx::launch_gemm_i8(m, n, k, a, w, k, mode, e, s));
    return WXH_OK;
  };
  {  // conv1: im2col rows of mel^T (f32ws), GELU, fp32 out into f32ws
    WXH_HIP(wx::launch_im2col_quant(E->f32ws, batch, T, C, 1, T, E->aq, E->k1p, E->asc, s));
    wx::EpiParams e;
    e.out = E->f32ws;
    e.ldo = d;
    e.bias = E->conv1_b;
    if (int r = gemm(batch * T, d, E->k1p, E->conv1_q, E->conv1_s, wx::EPI_F32_GELU, e)) return r;
    if (int r = mark(ST_CONV1)) return r;
  }
  {  // conv2: stride-2 im2col rows of the conv1 output, GELU, + positional embedding
    WXH_HIP(wx::launch_im2col_quant(E->f32ws, batch, T, d, 2, ctx, E->aq, 3 * d, E->asc, s));
    wx::EpiParams e;
    e.out = E->x;
    e.ldo = d;
    e.bias = E->conv2_b;
    e.aux = E->pos;
    e.rows_per_batch = ctx;
    if (int r = gemm(M, d, 3 * d, E->conv2_q, E->conv2_s, wx::EPI_CONV2, e)) return r;
    if (int r = mark(ST_CONV2)) return r;
  }
  const float scale = 1.0f / 8.0f;  // (hd^-1/4)^2 with hd = 64
  for (int l = 0; l < D.n_layer; ++l) {
    const LayerW& W = E->layers[l];
    WXH_HIP(wx::launch_layernorm(E->x, wx::DT_F32, d, nullptr, 0, nullptr, 0, W.ln1_g,
                                 W.ln1_b, 1e-5f, E->aq, wx::DT_I8, d, M, d, false, s,
                                 E->asc));
    if (int r = mark(ST_LN)) return r;
    {
      wx::EpiParams e;
      e.bias = W.bqkv;
      e.q = E->q;
      e.k = E->k;
      e.vt = E->vt;
      e.n_head = nh;
      e.t_pad = tp;
      e.d_model = d;
      e.rows_per_batch = ctx;
      e.q_scale = wx::attn_q_scale(scale);
      if (int r = gemm(M, 3 * d, d, W.wqkv_q, W.sqkv, wx::EPI_QKV, e)) return r;
      if (int r = mark(ST_QKV)) return r;
    }
    WXH_HIP(wx::launch_attention(E->q, E->k, E->vt, batch, nh, ctx, scale, E->f32ws,
                                 wx::DT_F32, d, s, true, E->tune_attn_keysplit));
    if (int r = mark(ST_ATTN)) return r;
    {
      WXH_HIP(wx::launch_quantize_rows(E->f32ws, wx::DT_F32, d, M, d, E->aq, d, d, E->asc,
                                       false, s));
      wx::EpiParams e;
      e.out = E->x;
      e.ldo = d;
      e.bias = W.bo;
      if (int r = gemm(M, d, d, W.wo_q, W.so, wx::EPI_RESID, e)) return r;
      if (int r = mark(ST_OUT)) return r;
    }
    WXH_HIP(wx::launch_layernorm(E->x, wx::DT_F32, d, nullptr, 0, nullptr, 0, W.ln2_g,
                                 W.ln2_b, 1e-5f, E->aq, wx::DT_I8, d, M, d, false, s,
                                 E->asc));
    if (int r = mark(ST_LN)) return r;
    {
      wx::EpiParams e;
      e.out = E->f32ws;
      e.ldo = ffn;
      e.bias = W.b1;
      if (int r = gemm(M, ffn, d, W.w1_q, W.s1, wx::EPI_F32_GELU, e)) return r;
      if (int r = mark(ST_FC1)) return r;
    }
    {
      WXH_HIP(wx::launch_quantize_rows(E->f32ws, wx::DT_F32, ffn, M, ffn, E->aq, ffn, ffn,
                                       E->asc, false, s));
      wx::EpiParams e;
      e.out = E->x;
      e.ldo = d;
      e.bias = W.b2;
      if (int r = gemm(M, d, ffn, W.w2_q, W.s2, wx::EPI_RESID, e)) return r;
      if (int r = mark(ST_FC2)) return r;
    }
  }
  return WXH_OK;
}

int run_body(wxh_encoder* E, int batch, int frames, hipStream_t s, StageTimer* timer) {
  if (E->i8) return run_body_i8(E, batch, frames, s, timer);
  const auto& D = E->dims;
  const int d = D.d_model, nh = D.n_head, T = frames;
  const int ctx = (T - 1) / 2 + 1;
  const int tp = wx::attn_padded_len(ctx);
  const int M = batch * ctx;
  const int conv_gelu = D.conv_gelu == WXH_GELU_POLY4_RNE ? wx::GELU_POLY4_RNE : wx::GELU_ERF;
  auto mark = [&](int stage) -> int {
    if (!timer) return WXH_OK;
    hipEvent_t ev;
    WXH_HIP(hipEventCreate(&ev));
    WXH_HIP(hipEventRecord(ev, s));
    timer->marks.push_back({stage, ev});
    return WXH_OK;
  };

  {  // conv1: window of 3 padded mel rows, GELU, into padded x1 rows
    wx::GemmA a{E->melT, D.n_mels, T, (int64_t)(T + 2) * D.n_mels};
    wx::EpiParams e;
    e.out = E->x1;
    e.ldo = d;
    e.bias = E->conv1_b;
    e.gelu = conv_gelu;
    e.rows_per_batch = T;
    e.out_batch_stride = (int64_t)(T + 2) * d;
    WXH_HIP(wx::launch_gemm(batch * T, d, 3 * D.n_mels, a, E->conv1_w, 3 * D.n_mels,
                            wx::EPI_CONV1, e, s));
    if (int r = mark(ST_CONV1)) return r;
  }
  {  // conv2: stride-2 window of 3 padded x1 rows, GELU, + positional embedding
    wx::GemmA a{E->x1, 2 * (int64_t)d, ctx, (int64_t)(T + 2) * d};
    wx::EpiParams e;
    e.out = E->x;
    e.ldo = d;
    e.bias = E->conv2_b;
    e.gelu = conv_gelu;
    e.aux = E->pos;
    e.rows_per_batch = ctx;
    set_splitk(E, e);
    WXH_HIP(wx::launch_gemm(M, d, 3 * d, a, E->conv2_w, 3 * d, wx::EPI_CONV2, e, s));
    if (int r = mark(ST_CONV2)) return r;
  }
  const float scale = 1.0f / 8.0f;  // (hd^-1/4)^2 with hd = 64
  for (int l = 0; l < D.n_layer; ++l) {
    const LayerW& W = E->layers[l];
    WXH_HIP(wx::launch_layernorm(E->x, wx::DT_F32, d, nullptr, 0, nullptr, 0, W.ln1_g,
                                 W.ln1_b, 1e-5f, E->h, wx::DT_BF16, d, M, d, kEncLnStream, s));
    if (int r = mark(ST_LN)) return r;
    {
      wx::GemmA a{E->h, d, M, 0};
      wx::EpiParams e;
      e.bias = W.bqkv;
      e.q = E->q;
      e.k = E->k;
      e.vt = E->vt;
      e.n_head = nh;
      e.t_pad = tp;
      e.d_model = d;
      e.rows_per_batch = ctx;
      e.q_scale = wx::attn_q_scale(scale);
      WXH_HIP(wx::launch_gemm(M, 3 * d, d, a, W.wqkv, d, wx::EPI_QKV, e, s));
      if (int r = mark(ST_QKV)) return r;
    }
    WXH_HIP(wx::launch_attention(E->q, E->k, E->vt, batch, nh, ctx, scale, E->o,
                                 wx::DT_BF16, d, s, true, E->tune_attn_keysplit));
    if (int r = mark(ST_ATTN)) return r;
    {
      wx::GemmA a{E->o, d, M, 0};
      wx::EpiParams e;
      e.out = E->x;
      e.ldo = d;
      e.bias = W.bo;
      set_splitk(E, e);
      WXH_HIP(wx::launch_gemm(M, d, d, a, W.wo, d, wx::EPI_RESID, e, s));
      if (int r = mark(ST_OUT)) return r;
    }
    WXH_HIP(wx::launch_layernorm(E->x, wx::DT_F32, d, nullptr, 0, nullptr, 0, W.ln2_g,
                                 W.ln2_b, 1e-5f, E->h, wx::DT_BF16, d, M, d, kEncLnStream, s));
    if (int r = mark(ST_LN)) return r;
    {
      wx::GemmA a{E->h, d, M, 0};
      wx::EpiParams e;
      e.out = E->f;
      e.ldo = E->ffn;
      e.bias = W.b1;
      e.gelu = D.mlp_gelu == WXH_GELU_POLY4_RNE ? wx::GELU_POLY4_RNE : wx::GELU_ERF;
      WXH_HIP(wx::launch_gemm(M, E->ffn, d, a, W.w1, d, wx::EPI_BF16, e, s));
      if (int r = mark(ST_FC1)) return r;
    }
    {
      wx::GemmA a{E->f, E->ffn, M, 0};
      wx::EpiParams e;
      e.out = E->x;
      e.ldo = d;
      e.bias = W.b2;
      set_splitk(E, e);
      WXH_HIP(wx::launch_gemm(M, d, E->ffn, a, W.w2, E->ffn, wx::EPI_RESID, e, s));
      if (int r = mark(ST_FC2)) return r;
    }
  }
  return WXH_OK;
}

int check_forward_args(wxh_encoder* E, int batch, int frames) {
  if (!E) return fail(WXH_ERR_INVALID, "encoder: null handle");
  if (int r = check_ctx(E->ctx, WXH_FAIL_ENCODER, "wxh_encoder_forward")) return r;
  if (wxh_encoder_ready(E) != WXH_OK) return WXH_ERR_STATE;
  WXH_REQUIRE(batch > 0 && frames >= 3, "encoder: batch=%d n_frames=%d", batch, frames);
  const int ctx = (frames - 1) / 2 + 1;
  WXH_REQUIRE(ctx <= E->dims.n_ctx,
              "encoder: n_frames=%d gives ctx=%d > positional embedding %d", frames,
              ctx, E->dims.n_ctx);
  return WXH_OK;
}

int forward_impl(wxh_encoder* E, const float* mel, int batch, int frames, float* out,
                 hipStream_t s, StageTimer* timer) {
  const auto& D = E->dims;
  const int ctx = (frames - 1) / 2 + 1;
  if (int r = ensure_workspace(E, batch, frames)) return r;
  if (E->done_pending && s != E->last_stream) WXH_HIP(hipStreamWaitEvent(s, E->done, 0));
  if (E->i8) {
    WXH_HIP(wx::launch_transpose_f32(mel, batch, D.n_mels, frames, E->f32ws, s));
  } else {
    // also zeroes the pad rows of the conv1 output, which conv2 reads
    WXH_HIP(wx::launch_prep_mel(mel, batch, D.n_mels, frames, E->melT, s, E->x1, D.d_model));
  }
  if (timer) {
    hipEvent_t ev;
    WXH_HIP(hipEventCreate(&ev));
    WXH_HIP(hipEventRecord(ev, s));
    timer->marks.push_back({ST_PREP, ev});
  }
  if (E->use_graph && !timer) {
    auto key = std::make_pair(batch, frames);
    auto it = E->graphs.find(key);
    if (it == E->graphs.end()) {
      // capture on the context's stream (recording only, nothing runs);
      // the instantiated graph is then launched on `s`
      hipStream_t cs = E->ctx->stream;
      WXH_HIP(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal));
      int r = run_body(E, batch, frames, cs, nullptr);
      hipGraph_t g = nullptr;
      hipError_t ee = hipStreamEndCapture(cs, &g);
      if (r != WXH_OK) {
        if (g) (void)hipGraphDestroy(g);
        return r;
      }
      if (ee != hipSuccess)
        return fail(WXH_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ee));
      hipGraphExec_t ex = nullptr;
      ee = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (ee != hipSuccess)
        return fail(WXH_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ee));
      it = E->graphs.emplace(key, ex).first;
    }
    WXH_HIP(hipGraphLaunch(it->second, s));
  } else {
    if (int r = run_body(E, batch, frames, s, timer)) return r;
  }
  WXH_HIP(wx::launch_layernorm(E->x, wx::DT_F32, D.d_model, nullptr, 0, nullptr, 0,
                               E->lnp_g, E->lnp_b, 1e-5f, out, wx::DT_F32, D.d_model,
                               batch * ctx, D.d_model, kEncLnStream, s));
  if (timer) {
    hipEvent_t ev;
    WXH_HIP(hipEventCreate(&ev));
    WXH_HIP(hipEventRecord(ev, s));
    timer->marks.push_back({ST_LNPOST, ev});
  }
  WXH_HIP(hipEventRecord(E->done, s));
  E->done_pending = true;
  E->last_stream = s;
  return WXH_OK;
}

// Pinned host and device staging of wxh_encoder_forward_host, grown (after
// the last forward has finished with them) to n_in / n_out floats.
int ensure_io_staging(wxh_encoder* E, size_t n_in, size_t n_out) {
  if (n_in <= E->cap_io_in && n_out <= E->cap_io_out) return WXH_OK;
  if (int r = quiesce(E, "wxh_encoder_forward_host staging regrow")) return r;
  if (n_in > E->cap_io_in) {
    if (E->h_mel) (void)hipHostFree(E->h_mel);
    if (E->d_mel) (void)hipFree(E->d_mel);
    E->h_mel = E->d_mel = nullptr;
    E->cap_io_in = 0;
    WXH_HIP(hipHostMalloc((void**)&E->h_mel, n_in * sizeof(float), hipHostMallocDefault));
    WXH_HIP(hipMalloc(&E->d_mel, n_in * sizeof(float)));
    E->cap_io_in = n_in;
  }
  if (n_out > E->cap_io_out) {
    if (E->h_out) (void)hipHostFree(E->h_out);
    if (E->d_out) (void)hipFree(E->d_out);
    E->h_out = E->d_out = nullptr;
    E->cap_io_out = 0;
    WXH_HIP(hipHostMalloc((void**)&E->h_out, n_out * sizeof(float), hipHostMallocDefault));
    WXH_HIP(hipMalloc(&E->d_out, n_out * sizeof(float)));
    E->cap_io_out = n_out;
  }
  return WXH_OK;
}

}  // namespace

extern "C" {

int wxh_encoder_create(wxh_ctx* c, const wxh_encoder_dims* dims, wxh_encoder** out) {
  if (int r = check_ctx(c, 0, "wxh_encoder_create")) return r;
  WXH_REQUIRE(dims && out, "wxh_encoder_create: null argument");
  const auto& D = *dims;
  WXH_REQUIRE(D.n_head > 0 && D.d_model == D.n_head * 64,
              "wxh_encoder_create: d_model=%d must be n_head*64 (n_head=%d)", D.d_model,
              D.n_head);
  WXH_REQUIRE(D.n_mels > 0 && D.n_mels % 8 == 0, "wxh_encoder_create: n_mels=%d", D.n_mels);
  WXH_REQUIRE(D.n_layer >= 0 && D.n_ctx > 0, "wxh_encoder_create: n_layer/n_ctx");
  WXH_REQUIRE(D.d_model <= wx::kMaxRowCols, "wxh_encoder_create: d_model too large");
  WXH_REQUIRE(D.mlp_gelu == WXH_GELU_ERF || D.mlp_gelu == WXH_GELU_POLY4_RNE,
              "wxh_encoder_create: mlp_gelu must be ERF or POLY4_RNE");
  WXH_REQUIRE(D.conv_gelu == WXH_GELU_ERF || D.conv_gelu == WXH_GELU_POLY4_RNE,
              "wxh_encoder_create: conv_gelu must be ERF or POLY4_RNE");
  hipEvent_t done = nullptr;
  WXH_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
  auto* E = new wxh_encoder;
  E->ctx = c;
  E->dims = D;
  E->done = done;
  E->tune_splitk = c->tune_splitk;
  E->tune_attn_keysplit = c->tune_attn_keysplit;
  E->ffn = 4 * D.d_model;
  const int d = D.d_model, ffn = E->ffn;
  auto& A = E->allocs;
  int r = WXH_OK;
  r = r ? r : dalloc(A, &E->conv1_w, (size_t)d * 3 * D.n_mels, true);
  r = r ? r : dalloc(A, &E->conv2_w, (size_t)d * 3 * d, true);
  r = r ? r : dalloc(A, &E->conv1_b, d, true);
  r = r ? r : dalloc(A, &E->conv2_b, d, true);
  r = r ? r : dalloc(A, &E->pos, (size_t)D.n_ctx * d, true);
  r = r ? r : dalloc(A, &E->lnp_g, d, true);
  r = r ? r : dalloc(A, &E->lnp_b, d, true);
  E->layers.resize(D.n_layer);
  for (auto& W : E->layers) {
    r = r ? r : dalloc(A, &W.wqkv, (size_t)3 * d * d, true);
    r = r ? r : dalloc(A, &W.wo, (size_t)d * d, true);
    r = r ? r : dalloc(A, &W.w1, (size_t)ffn * d, true);
    r = r ? r : dalloc(A, &W.w2, (size_t)d * ffn, true);
    r = r ? r : dalloc(A, &W.bqkv, 3 * d, true);
    r = r ? r : dalloc(A, &W.bo, d, true);
    r = r ? r : dalloc(A, &W.b1, ffn, true);
    r = r ? r : dalloc(A, &W.b2, d, true);
    r = r ? r : dalloc(A, &W.ln1_g, d, true);
    r = r ? r : dalloc(A, &W.ln1_b, d, true);
    r = r ? r : dalloc(A, &W.ln2_g, d, true);
    r = r ? r : dalloc(A, &W.ln2_b, d, true);
  }
  if (r != WXH_OK) {
    free_list(E->allocs);
    (void)hipEventDestroy(E->done);
    delete E;
    return r;
  }
  c->refs.fetch_add(1);
  *out = E;
  return WXH_OK;
}

int wxh_encoder_destroy(wxh_encoder* E) {
  if (!E) return WXH_OK;
  (void)hipSetDevice(E->ctx->device);
  (void)quiesce(E, "wxh_encoder_destroy", false);
  (void)hipStreamSynchronize(E->ctx->stream);
  drop_graphs(E);
  free_list(E->ws_allocs);
  free_list(E->allocs);
  if (E->stage) (void)hipFree(E->stage);
  if (E->h_mel) (void)hipHostFree(E->h_mel);
  if (E->h_out) (void)hipHostFree(E->h_out);
  if (E->d_mel) (void)hipFree(E->d_mel);
  if (E->d_out) (void)hipFree(E->d_out);
  (void)hipEventDestroy(E->done);
  wxh_ctx* c = E->ctx;
  delete E;
  ctx_release(c);
  return WXH_OK;
}

int wxh_encoder_set_weight(wxh_encoder* E, const char* name, const float* host,
                           const int64_t* shape, int ndim) {
  WXH_REQUIRE(E && name && host && shape, "wxh_encoder_set_weight: null argument");
  if (int r = check_ctx(E->ctx, 0, "wxh_encoder_set_weight")) return r;
  if (int r = quiesce(E, "wxh_encoder_set_weight", false)) return r;  // a forward may read it
  std::string n = name;
  if (n.rfind("w.", 0) == 0) n = n.substr(2);
  const auto& D = E->dims;
  const int64_t d = D.d_model, ffn = E->ffn, C = D.n_mels;
  auto bad_shape = [&]() {
    return fail(WXH_ERR_INVALID, "wxh_encoder_set_weight: %s has the wrong shape", name);
  };
  int r = WXH_OK;
  if (n == "conv1.weight" || n == "conv2.weight") {
    const int64_t cin = n == "conv1.weight" ? C : d;
    if (!shape_is(shape, ndim, {d, cin, 3})) return bad_shape();
    // (O, C, 3) -> [O][j*C + c]: tap-major K so a window of 3 rows is contiguous
    std::vector<float> perm((size_t)d * 3 * cin);
    for (int64_t o = 0; o < d; ++o)
      for (int64_t c = 0; c < cin; ++c)
        for (int64_t j = 0; j < 3; ++j)
          perm[(size_t)o * 3 * cin + j * cin + c] = host[(o * cin + c) * 3 + j];
    const bool c1 = n == "conv1.weight";
    r = upload_bf16(E, c1 ? E->conv1_w : E->conv2_w, perm.data(), (int)d, (int)(3 * cin),
                    E->i8_weights ? (c1 ? E->conv1_q : E->conv2_q) : nullptr,
                    c1 ? E->conv1_s : E->conv2_s, c1 ? E->k1p : (int)(3 * d));
  } else if (n == "conv1.bias" || n == "conv2.bias" || n == "ln_post.weight" ||
             n == "ln_post.bias") {
    if (!shape_is(shape, ndim, {d})) return bad_shape();
    float* dst = n == "conv1.bias" ? E->conv1_b
                 : n == "conv2.bias" ? E->conv2_b
                 : n == "ln_post.weight" ? E->lnp_g
                                         : E->lnp_b;
    r = upload_f32(E, dst, host, d);
  } else if (n == "positional_embedding") {
    if (!shape_is(shape, ndim, {D.n_ctx, d})) return bad_shape();
    r = upload_f32(E, E->pos, host, (size_t)D.n_ctx * d);
  } else if (n.rfind("blocks.", 0) == 0) {
    const size_t dot = n.find('.', 7);
    if (dot == std::string::npos) return fail(WXH_ERR_INVALID, "bad name %s", name);
    const int L = std::atoi(n.substr(7, dot - 7).c_str());
    if (L < 0 || L >= D.n_layer)
      return fail(WXH_ERR_INVALID, "wxh_encoder_set_weight: %s: layer out of range", name);
    const std::string t = n.substr(dot + 1);
    LayerW& W = E->layers[L];
    if (t == "attn.query.weight" || t == "attn.key.weight" || t == "attn.value.weight") {
      if (!shape_is(shape, ndim, {d, d})) return bad_shape();
      const int part = t == "attn.query.weight" ? 0 : t == "attn.key.weight" ? 1 : 2;
      r = upload_bf16(E, W.wqkv + (size_t)part * d * d, host, (int)d, (int)d,
                      E->i8_weights ? W.wqkv_q + (size_t)part * d * d : nullptr,
                      W.sqkv + part * d, (int)d);
    } else if (t == "attn.query.bias" || t == "attn.value.bias") {
      if (!shape_is(shape, ndim, {d})) return bad_shape();
      r = upload_f32(E, W.bqkv + (t == "attn.query.bias" ? 0 : 2 * d), host, d);
    } else if (t == "attn.out.weight") {
      if (!shape_is(shape, ndim, {d, d})) return bad_shape();
      r = upload_bf16(E, W.wo, host, (int)d, (int)d, E->i8_weights ? W.wo_q : nullptr, W.so,
                      (int)d);
    } else if (t == "mlp.0.weight") {
      if (!shape_is(shape, ndim, {ffn, d})) return bad_shape();
      r = upload_bf16(E, W.w1, host, (int)ffn, (int)d, E->i8_weights ? W.w1_q : nullptr, W.s1,
                      (int)d);
    } else if (t == "mlp.2.weight") {
      if (!shape_is(shape, ndim, {d, ffn})) return bad_shape();
      r = upload_bf16(E, W.w2, host, (int)d, (int)ffn, E->i8_weights ? W.w2_q : nullptr, W.s2,
                      (int)ffn);
    } else if (t == "mlp.0.bias") {
      if (!shape_is(shape, ndim, {ffn})) return bad_shape();
      r = upload_f32(E, W.b1, host, ffn);
    } else {
      float* dst = t == "attn.out.bias"    ? W.bo
                   : t == "mlp.2.bias"     ? W.b2
                   : t == "attn_ln.weight" ? W.ln1_g
                   : t == "attn_ln.bias"   ? W.ln1_b
                   : t == "mlp_ln.weight"  ? W.ln2_g
                   : t == "mlp_ln.bias"    ? W.ln2_b
                                           : nullptr;
      if (!dst) return fail(WXH_ERR_INVALID, "wxh_encoder_set_weight: unknown name %s", name);
      if (!shape_is(shape, ndim, {d})) return bad_shape();
      r = upload_f32(E, dst, host, d);
    }
  } else {
    return fail(WXH_ERR_INVALID, "wxh_encoder_set_weight: unknown name %s", name);
  }
  if (r == WXH_OK) E->have[n] = true;
  return r;
}

int wxh_encoder_ready(wxh_encoder* E) {
  WXH_REQUIRE(E, "wxh_encoder_ready: null handle");
  for (const auto& n : required_names(E->dims))
    if (!E->have.count(n))
      return fail(WXH_ERR_STATE, "encoder: weight %s has not been set", n.c_str());
  return WXH_OK;
}

int wxh_encoder_set_graph(wxh_encoder* E, int enabled) {
  WXH_REQUIRE(E, "wxh_encoder_set_graph: null handle");
  E->use_graph = enabled != 0;
  return WXH_OK;
}

int wxh_encoder_enable_int8(wxh_encoder* E) {
  WXH_REQUIRE(E, "wxh_encoder_enable_int8: null handle");
  if (E->i8_weights) return WXH_OK;
  const auto& D = E->dims;
  if (!E->have.empty())
    return fail(WXH_ERR_STATE, "wxh_encoder_enable_int8: call it before setting weights");
  if (D.d_model % wx::kI8KAlign != 0)
    return fail(WXH_ERR_UNSUPPORTED, "wxh_encoder_enable_int8: d_model=%d is not a multiple "
                "of %d", D.d_model, wx::kI8KAlign);
  if (D.mlp_gelu != WXH_GELU_ERF || D.conv_gelu != WXH_GELU_ERF)
    return fail(WXH_ERR_UNSUPPORTED, "wxh_encoder_enable_int8: needs the erf MLP and conv GELUs");
  const int d = D.d_model, ffn = E->ffn;
  E->k1p = (3 * D.n_mels + wx::kI8KAlign - 1) / wx::kI8KAlign * wx::kI8KAlign;
  auto& A = E->allocs;
  int r = WXH_OK;
  r = r ? r : dalloc(A, &E->conv1_q, (size_t)d * E->k1p, true);
  r = r ? r : dalloc(A, &E->conv2_q, (size_t)d * 3 * d, true);
  r = r ? r : dalloc(A, &E->conv1_s, d, true);
  r = r ? r : dalloc(A, &E->conv2_s, d, true);
  for (auto& W : E->layers) {
    r = r ? r : dalloc(A, &W.wqkv_q, (size_t)3 * d * d, true);
    r = r ? r : dalloc(A, &W.wo_q, (size_t)d * d, true);
    r = r ? r : dalloc(A, &W.w1_q, (size_t)ffn * d, true);
    r = r ? r : dalloc(A, &W.w2_q, (size_t)d * ffn, true);
    r = r ? r : dalloc(A, &W.sqkv, 3 * d, true);
    r = r ? r : dalloc(A, &W.so, d, true);
    r = r ? r : dalloc(A, &W.s1, ffn, true);
    r = r ? r : dalloc(A, &W.s2, d, true);
  }
  if (r != WXH_OK) return r;
  E->i8_weights = true;
  return WXH_OK;
}

int wxh_encoder_set_int8(wxh_encoder* E, int on) {
  WXH_REQUIRE(E, "wxh_encoder_set_int8: null handle");
  if (on && !E->i8_weights)
    return fail(WXH_ERR_STATE, "wxh_encoder_set_int8: wxh_encoder_enable_int8 was not called "
                "before the weights were set");
  if ((on != 0) != E->i8) {
    if (int r = quiesce(E, "wxh_encoder_set_int8", false)) return r;
    drop_graphs(E);
    E->i8 = on != 0;
  }
  return WXH_OK;
}

int wxh_encoder_forward(wxh_encoder* E, const float* mel, int batch, int frames,
                        float* out, void* stream) {
  if (int r = check_forward_args(E, batch, frames)) return r;
  WXH_REQUIRE(mel && out, "wxh_encoder_forward: null mel/out");
  return forward_impl(E, mel, batch, frames, out, pick(E->ctx, stream), nullptr);
}

int wxh_encoder_forward_host(wxh_encoder* E, const float* mel_host, int batch,
                             int frames, float* out_host) {
  if (int r = check_forward_args(E, batch, frames)) return r;
  WXH_REQUIRE(mel_host && out_host, "wxh_encoder_forward_host: null buffer");
  const auto& D = E->dims;
  const int ctx = (frames - 1) / 2 + 1;
  const size_t n_in = (size_t)batch * D.n_mels * frames;
  const size_t n_out = (size_t)batch * ctx * D.d_model;
  if (int r = ensure_io_staging(E, n_in, n_out)) return r;
  // a forward that timed out earlier may still be reading the staging
  if (int r = quiesce(E, "wxh_encoder_forward_host")) return r;
  hipStream_t s = E->ctx->stream;
  std::memcpy(E->h_mel, mel_host, n_in * sizeof(float));
  WXH_HIP(hipMemcpyAsync(E->d_mel, E->h_mel, n_in * sizeof(float), hipMemcpyHostToDevice, s));
  if (int r = forward_impl(E, E->d_mel, batch, frames, E->d_out, s, nullptr)) {
    (void)wait_stream(s, E->ctx->timeout_ms, "wxh_encoder_forward_host");
    return r;
  }
  WXH_HIP(hipMemcpyAsync(E->h_out, E->d_out, n_out * sizeof(float), hipMemcpyDeviceToHost, s));
  WXH_HIP(hipEventRecord(E->done, s));  // the copy out is part of this call
  E->done_pending = true;
  if (int r = quiesce(E, "wxh_encoder_forward_host")) return r;
  std::memcpy(out_host, E->h_out, n_out * sizeof(float));
  return WXH_OK;
}

int wxh_encoder_profile(wxh_encoder* E, const float* mel, int batch, int frames,
                        float* out, float* ms, int n) {
  if (int r = check_forward_args(E, batch, frames)) return r;
  WXH_REQUIRE(mel && out && ms && n >= 0, "wxh_encoder_profile: null argument");
  hipStream_t s = E->ctx->stream;
  StageTimer t;
  WXH_HIP(hipEventCreate(&t.start));
  WXH_HIP(hipEventRecord(t.start, s));
  int r = forward_impl(E, mel, batch, frames, out, s, &t);
  const int w = wait_stream(s, E->ctx->timeout_ms, "wxh_encoder_profile");
  const hipError_t e = w == WXH_OK ? hipSuccess : hipErrorNotReady;
  std::vector<float> acc(ST_COUNT, 0.f);
  hipEvent_t prev = t.start;
  for (auto& m : t.marks) {
    float dt = 0.f;
    if (r == WXH_OK && e == hipSuccess) (void)hipEventElapsedTime(&dt, prev, m.second);
    acc[m.first] += dt;
    prev = m.second;
  }
  for (auto& m : t.marks) (void)hipEventDestroy(m.second);
  (void)hipEventDestroy(t.start);
  if (r != WXH_OK) return r;
  if (w != WXH_OK) return w;
  for (int i = 0; i < n; ++i) ms[i] = i < ST_COUNT ? acc[i] : 0.f;
  return WXH_OK;
}

}  // extern "C"
