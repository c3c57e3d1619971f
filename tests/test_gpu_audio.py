"""The log-mel front end on the GPU (wxh_log_mel) against the oracle
(oracle/audio.py, float64 STFT), and audio -> features end to end.

Gate: |GPU - oracle| <= 1e-4 on the features (they span about [-1.5, 1.5];
the GPU runs the DFT and filterbank in fp64 and rounds once to fp32 before
the floor, so the differences are fp32 roundings, ~1e-7). A wrong window,
frame offset, reflection or filter is O(0.01-1).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import case, cosine, report
from oracle import audio as OA
from oracle import encoder as OE
from wxhip import _lib as L
from wxhip import synth

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 1e-4


def _clips():
    rng = np.random.default_rng(7)
    t = np.arange(OA.N_SAMPLES) / OA.SAMPLE_RATE
    speech = OA.pad_or_trim(OA.pcm16_to_float(np.load(GOLDEN / "jfk_3s.npy")))
    return [
        ("chirp+noise", (0.3 * np.sin(2 * np.pi * (100 * t + 120 * t * t))
                         + rng.normal(0, 0.05, OA.N_SAMPLES)).astype(np.float32)),
        ("jfk 3 s padded", speech),
        ("loud clipped noise", np.clip(rng.normal(0, 2, OA.N_SAMPLES), -1, 1).astype(np.float32)),
        ("silence", np.zeros(OA.N_SAMPLES, np.float32)),
    ]


@pytest.mark.parametrize("n_mels", [80, 128])
def test_log_mel_30s_windows(dev, n_mels):
    case(f"log-mel 30 s windows n_mels={n_mels}")
    for name, x in _clips():
        got = dev.log_mel(torch.from_numpy(x).to(dev.device), n_mels).cpu().numpy()
        want = OA.log_mel_spectrogram(x, n_mels)
        assert got.shape == want.shape == (n_mels, 3000), name
        err = float(np.abs(got - want).max())
        report(f"log_mel_{n_mels}", clip=name, max_abs=err)
        assert err <= TOL, (name, err)


def test_log_mel_batch_floor_per_clip_and_odd_lengths(dev):
    """A batch is the clips one by one (each floored at its own maximum);
    lengths that are not a multiple of the hop give len // 160 frames."""
    case("log-mel batch + odd lengths")
    clips = [x for _, x in _clips()[:3]]
    batch = torch.from_numpy(np.stack(clips)).to(dev.device)
    got = dev.log_mel(batch, 80).cpu().numpy()
    for b, x in enumerate(clips):
        assert np.abs(got[b] - OA.log_mel_spectrogram(x, 80)).max() <= TOL
    for n in (400, 401, 24000 + 77, 160 * 37):
        x = clips[1][:n]
        g = dev.log_mel(torch.from_numpy(np.ascontiguousarray(x)).to(dev.device), 80).cpu().numpy()
        w = OA.log_mel_spectrogram(x, 80)
        assert g.shape == w.shape == (80, n // 160) and np.abs(g - w).max() <= TOL, n


def test_whisper_api_and_fail_inject(dev):
    """wxhip.audio mirrors the whisper front-end entry points the reference
    calls: pad_or_trim and log_mel_spectrogram(samples, n_mels[, padding])."""
    from wxhip import audio as A
    case("log-mel whisper-style API")
    a = OA.pcm16_to_float(np.load(GOLDEN / "jfk_3s.npy"))
    with pytest.raises(TypeError):
        A.log_mel_spectrogram("clip.wav", n_mels=80, device=dev)
    padded = A.pad_or_trim(a)
    assert padded.shape == (A.N_SAMPLES,)
    m = A.log_mel_spectrogram(padded, n_mels=80, device=dev)
    assert tuple(m.shape) == (80, A.N_FRAMES)
    assert np.abs(m.cpu().numpy() - OA.log_mel_spectrogram(padded, 80)).max() <= TOL
    # padding= appends zero samples, as whisper's argument does
    m2 = A.log_mel_spectrogram(torch.from_numpy(a), n_mels=80, padding=A.N_SAMPLES - len(a),
                               device=dev)
    np.testing.assert_array_equal(m2.cpu().numpy(), m.cpu().numpy())
    dev.set_fail_inject(L.WXH_FAIL_FRONTEND)
    try:
        with pytest.raises(L.WxhError):
            dev.log_mel(torch.from_numpy(padded).to(dev.device), 80)
    finally:
        dev.set_fail_inject(0)


def test_audio_to_features_end_to_end(dev):
    """Audio -> GPU log-mel -> GPU encoder against oracle log-mel -> oracle
    encoder (tiny, 4 layers), on speech and on noise."""
    import wxhip
    case("audio -> features (tiny)")
    W = synth.make_weights("tiny")
    enc = wxhip.HipEncoder(dev, W)
    clips = [x for _, x in _clips()[:2]]
    got = enc.forward_audio(torch.from_numpy(np.stack(clips)).to(dev.device)).cpu().numpy()
    for b, x in enumerate(clips):
        ref = OE.encoder_torch(W, OA.log_mel_spectrogram(x, 80))
        c = cosine(got[b], ref)
        report("audio_to_features_tiny", clip=b, cosine=c)
        assert c >= 0.9999


def test_encode_recording_batches_windows(dev):
    """A 65 s recording at audio_ctx 500 (rung 512): three 30 s windows (the
    last 5 s), log-mel and encoder each in one batch, equal to running the
    windows one by one, and to the oracle front end + oracle encoder."""
    import wxhip
    from wxhip import windows as WN
    case("encode_recording 65 s, ctx 512 (tiny)")
    W = synth.make_weights("tiny")
    enc = wxhip.HipEncoder(dev, W)
    rng = np.random.default_rng(11)
    t = np.arange(65 * 16000) / 16000
    audio = (0.2 * np.sin(2 * np.pi * (200 + 30 * t) * t) + rng.normal(0, 0.03, t.size)).astype(np.float32)
    feats, ctx = WN.encode_recording(enc, audio, audio_ctx=500)
    assert ctx == 512 and tuple(feats.shape) == (3, 512, 384)
    got = feats.cpu().numpy()
    for i, (off, n) in enumerate(WN.split_windows(audio.size)):
        win = OA.pad_or_trim(audio[off:off + n])
        mel = dev.log_mel(torch.from_numpy(win).to(dev.device), 80)[None, :, :1024].contiguous()
        one = enc.forward(mel).cpu().numpy()[0]
        assert cosine(got[i], one) >= 0.99999
        ref = OE.encoder_torch(W, OA.log_mel_spectrogram(win, 80)[:, :1024])
        c = cosine(got[i], ref)
        report("encode_recording_tiny", window=i, cosine=c)
        assert c >= 0.9999
