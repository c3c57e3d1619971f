"""wxhip -- the Whisper encoder hot path on one MI355X (gfx950).

A drop-in for the XDNA path of drakosha/whisper-xdna: the reference's Python
surface (``encoder(W, mel, rt.matmul, ...)``, ``RawRT``, ``rowops``) backed by
libwxhip.so, hand-written HIP kernels driven through a C ABI (include/wxhip.h).

  wxhip.encoder   drop-in for src/npu_whisper_encoder.py (encoder() + helpers)
  wxhip.hiprt     HipRT (alias RawRT), drop-in for src/rawxrt.py
  wxhip.rowops    the row-op surface of src/rowops.py + compile_rowop.py codes
  wxhip.native    HipEncoder: the device-resident, hipGraph-replayed forward
  wxhip.device    Device: every kernel on torch device tensors
  wxhip.audio     WAV input and the log-mel front end (whisper names), on the GPU
  wxhip.windows   audio_ctx ladder and 30 s windows of long recordings, batched
  wxhip.weights   weights from dump_ref.py .npz files and openai-whisper checkpoints
  wxhip.synth     seeded synthetic weights / mels / row-op inputs
"""
from . import _lib
from ._lib import WxhError, WxhLibraryError
from .device import Device
from .hiprt import HipRT, RawRT
from .native import HipEncoder

__all__ = ["Device", "HipRT", "RawRT", "HipEncoder", "WxhError", "WxhLibraryError"]
