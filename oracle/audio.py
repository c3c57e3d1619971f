"""Whisper's log-mel front end, restated on the CPU (numpy, float64 STFT).

TEST INFRASTRUCTURE ONLY (see the package docstring).

The reference computes its encoder input with openai-whisper's
``pad_or_trim`` + ``log_mel_spectrogram`` (tools/dump_ref.py:55-57,
serve/npu_stt_server.py:334-336, bench/probe_int8_decode.py:128); its audio
comes from src/audio_io.py:15-44 (16-bit PCM, / 32768, channel mean).
openai-whisper is not vendored in the reference and not installed here; its
published algorithm (whisper/audio.py) is:

* 16 kHz audio, zero-padded or cut to 30 s (480000 samples);
* STFT with n_fft 400, hop 160, a periodic Hann window, frames centred
  (reflect padding of n_fft / 2 on both sides), the last frame dropped:
  480000 samples -> 3000 frames of 201 power bins |X_k|^2;
* a Slaney-style mel filterbank (librosa.filters.mel(sr=16000, n_fft=400,
  n_mels), Slaney area normalisation), restated in ``mel_filters``;
* log10 of max(mel power, 1e-10), floored at (its maximum - 8), then
  (x + 4) / 4.

Pinned in tests/test_oracle_audio.py against torch.stft (the routine whisper
calls), transformers' independent implementations of the filterbank and of
the whole feature extractor, and closed-form properties of the mel scale.
"""
import numpy as np

SAMPLE_RATE = 16000
N_FFT = 400
HOP_LENGTH = 160
N_SAMPLES = 30 * SAMPLE_RATE
N_FREQ = N_FFT // 2 + 1


def pcm16_to_float(raw_i16, n_channels=1):
    """int16 PCM -> float32 in [-1, 1), channels averaged (src/audio_io.py:30-33)."""
    a = np.asarray(raw_i16, dtype="<i2").astype(np.float32) / 32768.0
    if n_channels > 1:
        a = a.reshape(-1, n_channels).mean(axis=1)
    return a


def pad_or_trim(audio, length=N_SAMPLES):
    """Cut or zero-pad the last axis to `length` samples."""
    audio = np.asarray(audio, dtype=np.float32)
    if audio.shape[-1] > length:
        return audio[..., :length]
    pad = [(0, 0)] * (audio.ndim - 1) + [(0, length - audio.shape[-1])]
    return np.pad(audio, pad)


def hz_to_mel(f):
    """Slaney mel scale: linear (200/3 Hz per mel) below 1 kHz, logarithmic
    (27 mels per factor 6.4) above."""
    f = np.asarray(f, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    lin = f / f_sp
    return np.where(f >= min_log_hz,
                    min_log_mel + np.log(np.maximum(f, 1e-300) / min_log_hz) / logstep, lin)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)


def mel_filters(n_mels, sr=SAMPLE_RATE, n_fft=N_FFT):
    """[n_mels, n_fft/2 + 1] float32 triangular filters between mel-spaced
    edges from 0 Hz to sr/2, each scaled by 2 / (upper edge - lower edge) in Hz
    (Slaney normalisation), evaluated at the FFT bin frequencies in float64.
    As librosa.filters.mel does (the filters whisper ships were made with it),
    the triangle is stored as float32 before the float64 scale is applied and
    the product rounded to float32 again."""
    fft_f = np.linspace(0.0, sr / 2.0, n_fft // 2 + 1)
    edges = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sr / 2.0), n_mels + 2))
    fdiff = np.diff(edges)
    ramps = edges[:, None] - fft_f[None, :]
    w = np.zeros((n_mels, n_fft // 2 + 1), dtype=np.float32)
    for i in range(n_mels):
        lower = -ramps[i] / fdiff[i]
        upper = ramps[i + 2] / fdiff[i + 1]
        w[i] = np.maximum(0.0, np.minimum(lower, upper))
    w *= (2.0 / (edges[2:n_mels + 2] - edges[:n_mels]))[:, None]
    return w


def hann_periodic(n=N_FFT):
    return 0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n) / n)


def stft_power(audio):
    """|STFT|^2 of 1-D audio: [n_frames, 201] float64, n_frames = len // 160
    (centred frames, reflect padding, the last frame dropped)."""
    x = np.asarray(audio, dtype=np.float64)
    xp = np.pad(x, (N_FFT // 2, N_FFT // 2), mode="reflect")
    n_frames = 1 + (len(xp) - N_FFT) // HOP_LENGTH
    idx = np.arange(N_FFT)[None, :] + HOP_LENGTH * np.arange(n_frames)[:, None]
    spec = np.fft.rfft(xp[idx] * hann_periodic()[None, :], axis=1)
    return (spec.real ** 2 + spec.imag ** 2)[:-1]


def log_mel_spectrogram(audio, n_mels=80):
    """1-D audio (any length >= 201 samples) -> float32 [n_mels, len // 160]."""
    power = stft_power(audio)                                   # [frames, 201]
    mel = mel_filters(n_mels).astype(np.float64) @ power.T      # [n_mels, frames]
    log_spec = np.log10(np.maximum(mel, 1e-10))
    log_spec = np.maximum(log_spec, log_spec.max() - 8.0)
    return ((log_spec + 4.0) / 4.0).astype(np.float32)
