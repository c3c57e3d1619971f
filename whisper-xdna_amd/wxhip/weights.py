"""Encoder weights from the on-disk formats the reference uses.

* ``ref.npz`` as tools/dump_ref.py:72-86 writes it: ``mel`` and ``ref_out``
  (one sample's input and its torch reference output) plus ``"w." + key``
  for every entry of the encoder's state_dict, fp32. The reference reads it
  at src/npu_whisper_encoder.py:560-562 and serve/npu_stt_server.py:181-184.
* An openai-whisper checkpoint (the ``.pt`` that ``whisper.load_model``
  caches): a dict with ``dims`` and ``model_state_dict``, whose ``encoder.``
  entries are the same state_dict (serve/npu_stt_server.py:185-188 takes
  them with the same ``"w."`` prefix). A bare state_dict works too.

Only loaders that execute nothing from the file are used
(``numpy.load`` without pickles, ``torch.load(weights_only=True)``). The
result is the ``"w."``-keyed fp32 dict that ``HipEncoder`` uploads, rounding
to bf16 on the device, once.
"""
from pathlib import Path

import numpy as np


def load_ref_npz(path):
    """-> (W, mel or None, ref_out or None) from a dump_ref.py .npz."""
    with np.load(str(path), allow_pickle=False) as z:
        W = {k: np.ascontiguousarray(z[k], dtype=np.float32) for k in z.files}
    return W, W.pop("mel", None), W.pop("ref_out", None)


def save_ref_npz(path, W, mel=None, ref_out=None):
    """Write W (``"w."``-keyed) and optionally mel / ref_out in the same format."""
    out = {k: np.asarray(v, dtype=np.float32) for k, v in W.items()
           if k.startswith("w.") and isinstance(v, np.ndarray) and not k.endswith("_T")}
    if mel is not None:
        out["mel"] = np.asarray(mel, dtype=np.float32)
    if ref_out is not None:
        out["ref_out"] = np.asarray(ref_out, dtype=np.float32)
    np.savez(str(path), **out)


def encoder_state_to_w(state):
    """An encoder state_dict (keys ``encoder.<k>`` or ``<k>``, torch tensors or
    arrays) -> the ``"w."``-keyed fp32 dict; decoder entries are skipped."""
    W = {}
    has_prefix = any(k.startswith("encoder.") for k in state)
    for k, v in state.items():
        if has_prefix:
            if not k.startswith("encoder."):
                continue
            k = k[len("encoder."):]
        if hasattr(v, "detach"):
            v = v.detach().to("cpu").float().numpy()
        W["w." + k] = np.ascontiguousarray(v, dtype=np.float32)
    return W


def load_whisper_checkpoint(path):
    """-> (W, dims or None) from an openai-whisper checkpoint or a bare state_dict."""
    import torch
    ck = torch.load(str(path), map_location="cpu", weights_only=True)
    if isinstance(ck, dict) and "model_state_dict" in ck:
        return encoder_state_to_w(ck["model_state_dict"]), ck.get("dims")
    return encoder_state_to_w(ck), None


def load(path):
    """The weights of `path` by format: ``.npz`` (dump_ref.py) or a torch
    checkpoint. Returns the ``"w."``-keyed dict."""
    p = Path(path)
    if p.suffix == ".npz":
        return load_ref_npz(p)[0]
    return load_whisper_checkpoint(p)[0]
