"""Weights from the reference's on-disk formats (wxhip.weights): dump_ref.py's
.npz (tools/dump_ref.py:72-86) and an openai-whisper checkpoint's encoder
state_dict, through loaders that execute nothing from the file."""
import numpy as np
import pytest
import torch

from wxhip import synth
from wxhip import weights as WT


def _tiny():
    return {k: v for k, v in synth.make_weights("tiny").items() if isinstance(v, np.ndarray)}


def test_ref_npz_round_trip(tmp_path):
    W = _tiny()
    mel = np.random.default_rng(0).normal(size=(80, 3000)).astype(np.float32)
    p = tmp_path / "ref_tiny.npz"
    WT.save_ref_npz(p, W, mel=mel, ref_out=np.zeros((1500, 384), np.float32))
    W2, mel2, ref2 = WT.load_ref_npz(p)
    assert set(W2) == {k for k in W if k.startswith("w.") and not k.endswith("_T")}
    for k in W2:
        np.testing.assert_array_equal(W2[k], W[k])
    np.testing.assert_array_equal(mel2, mel)
    assert ref2.shape == (1500, 384)
    assert set(WT.load(p)) == set(W2)


def test_whisper_checkpoint_and_bare_state_dict(tmp_path):
    W = _tiny()
    enc_state = {k[2:]: torch.from_numpy(v) for k, v in W.items()
                 if k.startswith("w.") and not k.endswith("_T")}
    state = {"encoder." + k: v for k, v in enc_state.items()}
    state["decoder.token_embedding.weight"] = torch.zeros(8, 4)   # not the encoder's
    dims = {"n_mels": 80, "n_audio_ctx": 1500, "n_audio_state": 384, "n_audio_head": 6,
            "n_audio_layer": 4}
    ck = tmp_path / "tiny.pt"
    torch.save({"dims": dims, "model_state_dict": state}, ck)
    W2, d2 = WT.load_whisper_checkpoint(ck)
    assert d2 == dims and set(W2) == {"w." + k for k in enc_state}
    for k, v in enc_state.items():
        np.testing.assert_array_equal(W2["w." + k], v.numpy())
    bare = tmp_path / "bare.pt"
    torch.save(enc_state, bare)
    assert set(WT.load(bare)) == set(W2)


class _NotATensor:
    """An arbitrary class instance, which weights_only loading must refuse."""


def test_checkpoint_with_objects_is_refused(tmp_path):
    """weights_only loading: a pickled object in the file is an error, not code."""
    p = tmp_path / "object.pt"
    torch.save({"model_state_dict": {"encoder.x": torch.zeros(1)}, "extra": _NotATensor()}, p)
    with pytest.raises(Exception):
        WT.load_whisper_checkpoint(p)
