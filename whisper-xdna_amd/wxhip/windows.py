"""Variable context and windowing for long recordings, on the GPU.

The reference's server (serve/npu_stt_server.py) rounds a client's
``audio_ctx`` up onto a fixed ladder of contexts (LADDER and ``ctx_for``,
:61-72, 228-236), cuts a recording into 30 s windows, skips a tail shorter
than half a second (:430-440), and runs each window through pad_or_trim ->
log-mel -> encoder on ``mel[:, :2 * ctx]`` one after another (:331-343).

Here the same policy runs as one batch: every window's log-mel in one launch
(``Device.log_mel``), then one encoder forward over all windows at the
rung's context. HipEncoder keeps one hipGraph per (windows, frames) shape,
so a ladder of rungs is a bounded set of graphs, captured on first use or
ahead of time by ``warm``.
"""
import numpy as np

from .audio import HOP_LENGTH, N_SAMPLES, SAMPLE_RATE

LADDER = (512, 768, 1024, 1280, 1500)
DEFAULT_CTX = 1500


def ctx_for(requested, ladder=LADDER, default=DEFAULT_CTX):
    """Round a requested audio context up onto `ladder` (never less context
    than asked for; 0 or None means `default`; capped at the top rung)."""
    ladder = sorted(int(c) for c in ladder)
    if not ladder:
        raise ValueError("ladder is empty")
    req = int(requested) if requested else int(default)
    req = max(1, min(ladder[-1], req))
    for c in ladder:
        if req <= c:
            return c
    return ladder[-1]


def split_windows(n_samples, max_windows=0):
    """(offset, length) of each 30 s window of an `n_samples` recording; a
    tail under half a second after the first window is not speech and is
    dropped; `max_windows` > 0 caps the count."""
    out = []
    for off in range(0, max(n_samples, 1), N_SAMPLES):
        length = min(N_SAMPLES, n_samples - off)
        if off and length < SAMPLE_RATE // 2:
            break
        if max_windows and len(out) >= max_windows:
            break
        out.append((off, max(length, 0)))
    return out


def encode_recording(enc, audio, audio_ctx=None, ladder=LADDER, max_windows=0):
    """Features of every 30 s window of one recording, in one batch.

    enc: a HipEncoder; audio: 16 kHz fp32 samples (numpy or torch, any
    device). Returns (features [windows, ctx, d] on the GPU, ctx)."""
    import torch
    ctx = ctx_for(audio_ctx, ladder)
    if ctx > enc.n_ctx:
        raise ValueError(f"context {ctx} exceeds the model's {enc.n_ctx}")
    if not torch.is_tensor(audio):
        audio = torch.from_numpy(np.ascontiguousarray(audio, dtype=np.float32))
    audio = audio.to(device=enc.dev.device, dtype=torch.float32).reshape(-1)
    wins = split_windows(audio.numel(), max_windows)
    batch = torch.zeros(len(wins), N_SAMPLES, dtype=torch.float32, device=enc.dev.device)
    for i, (off, n) in enumerate(wins):
        batch[i, :n] = audio[off:off + n]
    mel = enc.dev.log_mel(batch, enc.n_mels)
    feats = enc.forward(mel[:, :, :2 * ctx].contiguous())
    return feats, ctx


def warm(enc, ladder=LADDER, windows=(1,)):
    """Capture the encoder graph of every rung (and window count) up front,
    as the server warms its overlays at start."""
    import torch
    for w in windows:
        for c in sorted(ladder):
            mel = torch.zeros(w, enc.n_mels, 2 * c, dtype=torch.float32, device=enc.dev.device)
            enc.forward(mel)
    torch.cuda.synchronize(enc.dev.device)


__all__ = ["LADDER", "DEFAULT_CTX", "ctx_for", "split_windows", "encode_recording", "warm",
           "HOP_LENGTH"]
