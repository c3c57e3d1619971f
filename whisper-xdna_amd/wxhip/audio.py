"""The log-mel front end, with the names the reference calls.

The reference turns 16 kHz samples into encoder input with openai-whisper's
``pad_or_trim`` + ``log_mel_spectrogram`` on the CPU (tools/dump_ref.py:55-57,
serve/npu_stt_server.py:334-336). Here the same two functions take the same
arguments; ``log_mel_spectrogram`` runs on the GPU (``wxh_log_mel``) and
returns a device tensor, ready for ``HipEncoder.forward``. Decoding audio
files (the reference's src/audio_io.py) is outside this path: callers pass
samples.
"""
import numpy as np

SAMPLE_RATE = 16000
N_FFT = 400
HOP_LENGTH = 160
CHUNK_LENGTH = 30
N_SAMPLES = CHUNK_LENGTH * SAMPLE_RATE   # 480000 samples in a 30 s window
N_FRAMES = N_SAMPLES // HOP_LENGTH      # 3000 mel frames

_dev = None


def pad_or_trim(array, length=N_SAMPLES, axis=-1):
    """Cut or zero-pad `axis` to `length` samples (numpy array or torch tensor)."""
    if hasattr(array, "detach"):
        import torch
        n = array.shape[axis]
        if n > length:
            return array.narrow(axis, 0, length)
        if n < length:
            pad = [0] * (2 * array.dim())
            pad[2 * (array.dim() - 1 - (axis % array.dim())) + 1] = length - n
            return torch.nn.functional.pad(array, pad)
        return array
    array = np.asarray(array)
    n = array.shape[axis]
    if n > length:
        return array.take(indices=range(length), axis=axis)
    if n < length:
        widths = [(0, 0)] * array.ndim
        widths[axis] = (0, length - n)
        return np.pad(array, widths)
    return array


def log_mel_spectrogram(audio, n_mels=80, padding=0, device=None):
    """Whisper's log-mel features on the GPU.

    audio: fp32 samples at 16 kHz ([n] or [B, n]; numpy or torch, any
    device); `padding` zero samples are appended first. Returns
    an fp32 torch tensor on the GPU, [n_mels, n // 160] (or [B, n_mels,
    n // 160]), each clip floored at its own maximum - 8.
    """
    import torch
    from .device import Device
    global _dev
    dev = device
    if dev is None:
        if _dev is None:
            _dev = Device(0)
        dev = _dev
    if isinstance(audio, (str, bytes)):
        raise TypeError("log_mel_spectrogram takes samples; decoding audio files is "
                        "outside this path")
    if not torch.is_tensor(audio):
        audio = torch.from_numpy(np.ascontiguousarray(audio, dtype=np.float32))
    audio = audio.to(device=dev.device, dtype=torch.float32)
    if padding > 0:
        audio = torch.nn.functional.pad(audio, (0, padding))
    return dev.log_mel(audio.contiguous(), n_mels)
