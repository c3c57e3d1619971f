"""wxh_log_mel_noalloc, the allocation-free front end, through the C ABI:
two calls in a row (the second with fewer clips, fewer samples and the other
mel count) each give exactly what wxh_log_mel gives on the same audio, and
the oracle's features within the front end's tolerance; batch and n_mels
outside the fixed scratch are refused before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import case
from oracle import audio as OA
from wxhip import _lib as L

pytestmark = pytest.mark.gpu

TOL = 1e-4   # the front end's gate against the oracle (tests/test_gpu_audio.py)


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _both(dev, audio, n_mels):
    """(wxh_log_mel_noalloc, wxh_log_mel) features of device audio [B, n]."""
    B, n = audio.shape
    outs = []
    for name in ("wxh_log_mel_noalloc", "wxh_log_mel"):
        out = torch.full((B, n_mels, n // 160), float("nan"), device=dev.device)
        rc = getattr(dev.lib, name)(dev.handle, _ptr(audio), B, n, n_mels, _ptr(out), dev.stream())
        assert rc == L.WXH_OK, (name, rc, dev.lib.wxh_last_error())
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def test_log_mel_noalloc_matches_log_mel(dev):
    rng = np.random.default_rng(42)
    case("wxh_log_mel_noalloc: 4 clips x 480000 samples, 128 mels")
    a = rng.normal(0, 0.1, (4, 480000)).astype(np.float32)
    a[2] *= 0                                   # a silent clip: its own floor
    got, want = _both(dev, torch.from_numpy(a).to(dev.device), 128)
    np.testing.assert_array_equal(got, want)
    assert np.abs(got[1] - OA.log_mel_spectrogram(a[1], 128)).max() <= TOL
    case("wxh_log_mel_noalloc: then 2 clips x 160037 samples, 80 mels")
    b = rng.normal(0, 0.3, (2, 160037)).astype(np.float32)
    got, want = _both(dev, torch.from_numpy(b).to(dev.device), 80)
    np.testing.assert_array_equal(got, want)
    assert np.abs(got[0] - OA.log_mel_spectrogram(b[0], 80)).max() <= TOL


def test_log_mel_noalloc_limits(dev):
    case("wxh_log_mel_noalloc: refusals (host side, nothing launched)")
    audio = torch.zeros(1, 480000, device=dev.device)
    out = torch.zeros(1, 96, 3000, device=dev.device)
    rc = dev.lib.wxh_log_mel_noalloc(dev.handle, _ptr(audio), 1, 480000, 96, _ptr(out),
                                     dev.stream())
    assert rc == L.WXH_ERR_UNSUPPORTED and b"80- and 128-mel" in dev.lib.wxh_last_error()
    rc = dev.lib.wxh_log_mel_noalloc(dev.handle, _ptr(audio), 257, 480000, 80, _ptr(out),
                                     dev.stream())
    assert rc == L.WXH_ERR_INVALID and b"256" in dev.lib.wxh_last_error()
