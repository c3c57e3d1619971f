"""The log-mel front end's oracle (oracle/audio.py) pinned on the CPU, and the
library's host-side filterbank checked against it.

Pins, chosen so that a dropped term, a wrong window, a wrong frame offset or
a mis-scaled filter fails one of them:
* torch.stft (the routine openai-whisper calls) on the same samples;
* transformers' mel_filter_bank and WhisperFeatureExtractor, an independent
  implementation of the same filterbank and of the whole feature pipeline;
* closed forms of the Slaney mel scale (linear below 1 kHz at 200/3 Hz per
  mel, 27 mels per factor 6.4 above) and of the filter shapes;
* the reference's own test audio (tests/data/jfk.wav, a 3 s excerpt in
  tests/golden/jfk_3s.npy) as real speech input.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import audio as OA

GOLDEN = Path(__file__).resolve().parent / "golden"


def _signals():
    rng = np.random.default_rng(5)
    t = np.arange(OA.N_SAMPLES) / OA.SAMPLE_RATE
    chirp = 0.3 * np.sin(2 * np.pi * (100 * t + 120 * t * t))
    noise = rng.normal(0, 0.05, OA.N_SAMPLES)
    speech = OA.pcm16_to_float(np.load(GOLDEN / "jfk_3s.npy"))
    return {
        "chirp+noise": (chirp + noise).astype(np.float32),
        "jfk 3 s padded to 30 s": OA.pad_or_trim(speech),
        "short 1.5 s tone": (0.5 * np.sin(2 * np.pi * 440 * t[:24000])).astype(np.float32),
    }


def test_stft_power_matches_torch_stft():
    for name, x in _signals().items():
        got = OA.stft_power(x)
        t = torch.stft(torch.from_numpy(x).double(), OA.N_FFT, OA.HOP_LENGTH,
                       window=torch.hann_window(OA.N_FFT, dtype=torch.float64),
                       return_complex=True)
        want = (t.abs() ** 2)[..., :-1].T.numpy()
        assert got.shape == (len(x) // OA.HOP_LENGTH, OA.N_FREQ) == want.shape, name
        assert np.abs(got - want).max() <= 1e-12 * want.max(), name


def test_mel_scale_closed_forms():
    assert OA.hz_to_mel(1000.0) == pytest.approx(15.0)
    assert OA.hz_to_mel(200.0 / 3) == pytest.approx(1.0)
    assert OA.hz_to_mel(6400.0) == pytest.approx(15.0 + 27.0)
    f = np.linspace(0, 8000, 1001)
    np.testing.assert_allclose(OA.mel_to_hz(OA.hz_to_mel(f)), f, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("n_mels", [80, 128])
def test_mel_filters_shape_and_independent_implementation(n_mels):
    w = OA.mel_filters(n_mels)
    assert w.shape == (n_mels, OA.N_FREQ) and w.dtype == np.float32 and (w >= 0).all()
    # each filter is one run of nonzero bins (a triangle), rising then falling
    for row in w:
        nz = np.nonzero(row)[0]
        assert len(nz) and (np.diff(nz) == 1).all()
        peak = nz[np.argmax(row[nz])]
        assert (np.diff(row[nz[0]:peak + 1]) >= 0).all() and (np.diff(row[peak:nz[-1] + 1]) <= 0).all()
    # Slaney normalisation: each triangle has unit area in Hz; sampled at the
    # 40 Hz bin spacing that holds to a few % for the filters spanning 6 or
    # more bins, 1 % on average (the narrow low ones are sampled at a handful
    # of points)
    area = w.sum(1) * 40.0
    wide = (w > 0).sum(1) >= 6
    assert wide.sum() >= 10 and np.abs(area[wide] - 1).max() < 0.03
    assert abs(area[wide].mean() - 1) < 0.01
    audio_utils = pytest.importorskip("transformers.audio_utils")
    fb = audio_utils.mel_filter_bank(num_frequency_bins=OA.N_FREQ, num_mel_filters=n_mels,
                                     min_frequency=0.0, max_frequency=8000.0,
                                     sampling_rate=OA.SAMPLE_RATE, norm="slaney",
                                     mel_scale="slaney").T
    assert np.abs(w - fb).max() <= 1e-6 * fb.max()


@pytest.mark.parametrize("n_mels", [80, 128])
def test_log_mel_matches_whisper_feature_extractor(n_mels):
    tf = pytest.importorskip("transformers")
    fe = tf.WhisperFeatureExtractor(feature_size=n_mels)
    for name, x in _signals().items():
        if len(x) != OA.N_SAMPLES:
            continue  # the extractor pads to 30 s itself; compare 30 s windows
        want = fe(x, sampling_rate=OA.SAMPLE_RATE, return_tensors="np")["input_features"][0]
        got = OA.log_mel_spectrogram(x, n_mels)
        assert got.shape == want.shape == (n_mels, 3000), name
        # the extractor runs its STFT in float32 (as whisper's torch.stft does)
        assert np.abs(got - want).max() < 1e-4, name


def test_log_mel_floor_and_range():
    x = _signals()["chirp+noise"]
    y = OA.log_mel_spectrogram(x, 80)
    # floor: nothing more than 8 decades (2.0 after the /4) below the maximum
    assert y.max() - y.min() <= 2.0 + 1e-6
    silence = OA.log_mel_spectrogram(np.zeros(OA.N_SAMPLES, np.float32), 80)
    np.testing.assert_allclose(silence, (-10 + 4) / 4, atol=1e-6)  # log10(1e-10)


def test_pad_or_trim_and_pcm16():
    a = np.arange(10, dtype=np.float32)
    assert OA.pad_or_trim(a, 4).tolist() == [0, 1, 2, 3]
    assert OA.pad_or_trim(a, 12).tolist() == list(range(10)) + [0, 0]
    pcm = np.array([0, 16384, -32768, 32767], np.int16)
    np.testing.assert_array_equal(OA.pcm16_to_float(pcm), [0, 0.5, -1, 32767 / 32768])


@pytest.mark.parametrize("n_mels", [80, 128])
def test_library_filterbank_equals_oracle(n_mels):
    """wxh_mel_filterbank (host code, no GPU) equals the oracle's filterbank
    exactly (same edges, same float32 rounding points; the oracle's zeros
    may carry numpy's sign)."""
    from wxhip import _lib as L
    lib = L.load()
    out = np.zeros((n_mels, OA.N_FREQ), np.float32)
    assert lib.wxh_mel_filterbank(n_mels, out.ctypes.data_as(C.c_void_p)) == 0
    np.testing.assert_array_equal(out, OA.mel_filters(n_mels))
