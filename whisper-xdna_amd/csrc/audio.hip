// Whisper's log-mel front end on the GPU: 16 kHz audio -> [n_mels, frames].
//
// Semantics (openai-whisper's log_mel_spectrogram, which the reference calls
// at tools/dump_ref.py:55-57 and serve/npu_stt_server.py:334-336):
// centred frames of n_fft = 400 samples every hop = 160 (reflect padding of
// 200 at both ends, the last frame dropped: n_samples / 160 frames), a
// periodic Hann window, power |X_k|^2 of the 201 real-input DFT bins, a
// Slaney mel filterbank (librosa.filters.mel(16000, 400, n_mels)), log10 of
// max(., 1e-10), floored at the clip's maximum - 8, then (x + 4) / 4.
//
// logmel_frame_kernel: one workgroup per (frame, clip). The windowed frame
// sits in LDS; thread k < 201 forms the power of bin k with the Goertzel
// recurrence in fp64 (fp64 FMA runs at the fp32 rate on this GPU, and it
// keeps the bins near the -8 floor exact); the filterbank rows and log10
// follow.
// logmel_norm_kernel: applies the floor at the clip maximum (reduced by the
// frame kernel) and the affine map in place, over a grid per clip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace wx {

constexpr int kNFFT = 400, kHop = 160, kNFreq = kNFFT / 2 + 1;

// Slaney mel scale (librosa's default, htk = False): 200/3 Hz per mel below
// 1 kHz, 27 mels per factor 6.4 above
static double hz_to_mel(double f) {
  const double f_sp = 200.0 / 3, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
  const double logstep = std::log(6.4) / 27.0;
  return f >= min_log_hz ? min_log_mel + std::log(f / min_log_hz) / logstep : f / f_sp;
}
static double mel_to_hz(double m) {
  const double f_sp = 200.0 / 3, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
  const double logstep = std::log(6.4) / 27.0;
  return m >= min_log_mel ? min_log_hz * std::exp(logstep * (m - min_log_mel)) : f_sp * m;
}

// [n_mels][201] float32 triangles between mel-spaced edges (0 Hz .. 8 kHz)
// at the bin frequencies 40 k Hz, Slaney area normalisation 2 / (f[i+2] -
// f[i]); the triangle is rounded to float32 before the scale and the product
// again, as librosa stores it.
std::vector<float> mel_filterbank(int n_mels) {
  std::vector<double> edges(n_mels + 2);
  const double top = hz_to_mel(8000.0), step = top / (n_mels + 1);  // numpy.linspace
  for (int i = 0; i < n_mels + 2; ++i) edges[i] = mel_to_hz(i == n_mels + 1 ? top : i * step);
  std::vector<float> w((size_t)n_mels * kNFreq);
  for (int i = 0; i < n_mels; ++i) {
    const double enorm = 2.0 / (edges[i + 2] - edges[i]);
    const double d0 = edges[i + 1] - edges[i], d1 = edges[i + 2] - edges[i + 1];
    for (int k = 0; k < kNFreq; ++k) {
      const double f = 40.0 * k;
      const double lower = -(edges[i] - f) / d0, upper = (edges[i + 2] - f) / d1;
      const float tri = (float)std::fmax(0.0, std::fmin(lower, upper));
      w[(size_t)i * kNFreq + k] = (float)((double)tri * enorm);
    }
  }
  return w;
}

// The device-side constants of one n_mels, in one buffer:
//   double cos(2 pi j / 400) [400], double periodic Hann [400],
//   int32 (first bin, bin count, weight offset) per mel filter [3 n_mels],
//   float the filters' nonzero weights, packed.
// Each triangle is nonzero on one run of bins and every bin lies in at most
// two of them, so the packed weights are ~2 x 201 floats instead of
// n_mels x 201.
std::vector<uint8_t> logmel_constants(int n_mels) {
  const std::vector<float> w = mel_filterbank(n_mels);
  std::vector<int32_t> meta(3 * n_mels);
  std::vector<float> packed;
  for (int m = 0; m < n_mels; ++m) {
    int lo = kNFreq, hi = -1;
    for (int k = 0; k < kNFreq; ++k)
      if (w[(size_t)m * kNFreq + k] != 0.f) {
        lo = lo < k ? lo : k;
        hi = k;
      }
    if (hi < lo) lo = 0, hi = -1;
    meta[3 * m] = lo;
    meta[3 * m + 1] = hi - lo + 1;
    meta[3 * m + 2] = (int32_t)packed.size();
    for (int k = lo; k <= hi; ++k) packed.push_back(w[(size_t)m * kNFreq + k]);
  }
  std::vector<uint8_t> buf(2 * kNFFT * sizeof(double) + meta.size() * 4 + packed.size() * 4);
  double* t = reinterpret_cast<double*>(buf.data());
  const double pi = 3.14159265358979323846;
  for (int j = 0; j < kNFFT; ++j) {
    t[j] = std::cos(2.0 * pi * j / kNFFT);
    t[kNFFT + j] = 0.5 - 0.5 * std::cos(2.0 * pi * j / kNFFT);
  }
  std::memcpy(buf.data() + 2 * kNFFT * sizeof(double), meta.data(), meta.size() * 4);
  std::memcpy(buf.data() + 2 * kNFFT * sizeof(double) + meta.size() * 4, packed.data(),
              packed.size() * 4);
  return buf;
}

// The clip maximum is reduced through kMaxSlots slots per clip: the frame
// kernel's workgroups atomic-max their frame's maximum into slot f % 64 (as
// an order-preserving int), which spreads the atomics; the normalisation
// grid reads the clip's 64 slots.
constexpr int kMaxSlots = kLogMelSlots;
__device__ __forceinline__ int ordered_key(float v) {
  const int i = __float_as_int(v);
  return i >= 0 ? i : i ^ 0x7fffffff;
}
__device__ __forceinline__ float ordered_val(int k) {
  return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff);
}

__global__ void logmel_init_kernel(int* __restrict__ slots, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) slots[i] = ordered_key(-INFINITY);
}

__global__ __launch_bounds__(256) void logmel_frame_kernel(
    const float* __restrict__ audio, int n_samples, int n_frames, int n_mels,
    const uint8_t* __restrict__ consts, float* __restrict__ out, int* __restrict__ slots) {
  __shared__ float red[4];
  const double* tables = reinterpret_cast<const double*>(consts);
  const int32_t* meta = reinterpret_cast<const int32_t*>(consts + 2 * kNFFT * sizeof(double));
  const float* filt = reinterpret_cast<const float*>(meta + 3 * n_mels);
  __shared__ double ct[kNFFT];
  __shared__ double xw[kNFFT];
  __shared__ double pw[kNFreq];
  const int f = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const float* x = audio + (int64_t)b * n_samples;
  for (int n = tid; n < kNFFT; n += blockDim.x) {
    ct[n] = tables[n];
    // centred frame: sample f * hop + n - n_fft / 2, reflected at both ends
    int j = f * kHop + n - kNFFT / 2;
    j = j < 0 ? -j : j;
    j = j >= n_samples ? 2 * (n_samples - 1) - j : j;
    xw[n] = (double)x[j] * tables[kNFFT + n];
  }
  __syncthreads();
  if (tid < kNFreq) {
    // |X_k|^2 by the Goertzel recurrence s_n = x_n + c s_{n-1} - s_{n-2},
    // c = 2 cos(2 pi k / N): |X_k|^2 = s1^2 + s2^2 - c s1 s2 with s1, s2 the
    // last two states. Two fp64 operations per sample and no twiddle index
    // arithmetic (which made a table-driven direct DFT instruction-bound).
    const double c = 2.0 * ct[tid];
    double s1 = 0.0, s2 = 0.0;
#pragma unroll 8
    for (int n = 0; n < kNFFT; ++n) {
      const double s0 = fma(c, s1, xw[n] - s2);
      s2 = s1;
      s1 = s0;
    }
    pw[tid] = fma(s1, s1 - c * s2, s2 * s2);
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int m = tid; m < n_mels; m += blockDim.x) {
    const int lo = meta[3 * m], len = meta[3 * m + 1];
    const float* fr = filt + meta[3 * m + 2];
    double s = 0.0;
    for (int k = 0; k < len; ++k) s = fma((double)fr[k], pw[lo + k], s);
    const float v = (float)log10(fmax(s, 1e-10));
    out[((int64_t)b * n_mels + m) * n_frames + f] = v;
    mx = fmaxf(mx, v);
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) {
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    atomicMax(slots + b * kMaxSlots + (f % kMaxSlots), ordered_key(mx));
  }
}

// floor at the clip maximum - 8, then (x + 4) / 4; grid (chunks, clips)
__global__ __launch_bounds__(256) void logmel_norm_kernel(float* __restrict__ out,
                                                          int64_t per_clip,
                                                          const int* __restrict__ slots) {
  const int b = blockIdx.y;
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxSlots; ++i) mx = fmaxf(mx, ordered_val(slots[b * kMaxSlots + i]));
  const float floor_v = mx - 8.0f;
  float* y = out + (int64_t)b * per_clip;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per_clip;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = (fmaxf(y[i], floor_v) + 4.0f) * 0.25f;
}

hipError_t launch_log_mel(const float* audio, int batch, int n_samples, int n_mels,
                          const uint8_t* consts, float* out, int* slots, hipStream_t s) {
  const int n_frames = n_samples / kHop;
  if (batch <= 0 || n_frames <= 0) return hipSuccess;
  const int ns = batch * kMaxSlots;
  logmel_init_kernel<<<(ns + 255) / 256, 256, 0, s>>>(slots, ns);
  logmel_frame_kernel<<<dim3(n_frames, batch), 256, 0, s>>>(audio, n_samples, n_frames, n_mels,
                                                             consts, out, slots);
  const int64_t per_clip = (int64_t)n_mels * n_frames;
  const int chunks = (int)std::min<int64_t>((per_clip + 2047) / 2048, 1024);
  logmel_norm_kernel<<<dim3(chunks, batch), 256, 0, s>>>(out, per_clip, slots);
  return hipGetLastError();
}

// ------------------------------------------------------------ allocation-free
// Everything launch_log_mel needs beyond its input and output, for callers
// that cannot allocate device memory, in one file-scope device array: the
// clip-maximum slots of up to kNoAllocClips clips, then the constants of the
// two filterbanks Whisper uses (80 and 128 mels). Each GPU the library runs
// on holds its own copy, 96 KiB, until the process ends. In host code
// `scratch` only names the symbol: its device address on each GPU comes from
// hipGetSymbolAddress, once per device at set-up, and only that address is
// ever handed to a kernel.
constexpr int kNoAllocConstBytes = 16 << 10;
constexpr int kNoAllocSlotBytes = kNoAllocClips * kMaxSlots * (int)sizeof(int);
constexpr int kNoAllocMels[2] = {80, 128};
static __device__ __align__(256) uint8_t scratch[kNoAllocSlotBytes + 2 * kNoAllocConstBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};  // per device: the address of `scratch` there
}  // namespace

hipError_t logmel_noalloc_setup(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  if (g_scratch[device]) return hipSuccess;
  void* base = nullptr;
  hipError_t e = hipGetSymbolAddress(&base, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  for (int i = 0; i < 2; ++i) {
    const std::vector<uint8_t> c = logmel_constants(kNoAllocMels[i]);
    if (c.size() > (size_t)kNoAllocConstBytes) return hipErrorInvalidValue;
    e = hipMemcpy(static_cast<uint8_t*>(base) + kNoAllocSlotBytes + i * kNoAllocConstBytes,
                  c.data(), c.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
  }
  g_scratch[device] = static_cast<uint8_t*>(base);
  return hipSuccess;
}

hipError_t launch_log_mel_noalloc(int device, const float* audio, int batch, int n_samples,
                                  int n_mels, float* out, hipStream_t s) {
  uint8_t* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device >= 0 && device < kMaxDevices) base = g_scratch[device];
  }
  const int which = n_mels == kNoAllocMels[0] ? 0 : n_mels == kNoAllocMels[1] ? 1 : -1;
  if (!base || which < 0 || batch > kNoAllocClips) return hipErrorInvalidValue;
  return launch_log_mel(audio, batch, n_samples, n_mels,
                        base + kNoAllocSlotBytes + which * kNoAllocConstBytes, out,
                        reinterpret_cast<int*>(base), s);
}

}  // namespace wx
