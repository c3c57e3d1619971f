"""Seeded synthetic encoder weights, log-mels and row-op inputs.

There is no network here and no checkpoint, so every workload is synthetic
but shaped exactly like the real model. Weights follow the
``"w." + state_dict`` naming of tools/dump_ref.py:72-76, so a dict loaded from
a real ``ref.npz`` drops in unchanged.

Draw order (fixed, so the CPU oracle and the GPU see identical values):
  rng = numpy.random.default_rng(seed)
  for each key in ``weight_keys(cfg)`` order that is a conv/linear weight or
  bias: ``rng.standard_normal(shape, dtype=float32) * float32(0.02)``
  LayerNorm gamma = 1, beta = 0 (no draw); the key projection has no bias;
  the positional embedding is whisper's fixed sinusoid table (no draw).
Mel: ``default_rng(seed).normal(-0.3, 0.5, (n_mels, n_frames))`` as float32,
clipped to [-1, 1.5]; batch item i uses seed i.
"""
import math

import numpy as np

# Encoder geometries of the shapes this path is measured on.
MODELS = {
    "tiny": dict(n_mels=80, d=384, n_head=6, n_layer=4, n_ctx=1500),
    "small": dict(n_mels=80, d=768, n_head=12, n_layer=12, n_ctx=1500),
    "large-v3": dict(n_mels=128, d=1280, n_head=20, n_layer=32, n_ctx=1500),
}


def sinusoids(length, channels, max_timescale=10000):
    """Whisper's positional embedding: [sin | cos] of a geometric frequency
    ladder (openai-whisper model.py ``sinusoids``; consumed at
    npu_whisper_encoder.py:456-458)."""
    assert channels % 2 == 0
    inc = math.log(max_timescale) / (channels // 2 - 1)
    inv = np.exp(-inc * np.arange(channels // 2, dtype=np.float64))
    t = np.arange(length, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1).astype(np.float32)


def weight_keys(n_layer):
    keys = ["conv1.weight", "conv1.bias", "conv2.weight", "conv2.bias"]
    for L in range(n_layer):
        p = f"blocks.{L}."
        keys += [p + k for k in (
            "attn_ln.weight", "attn_ln.bias",
            "attn.query.weight", "attn.query.bias", "attn.key.weight",
            "attn.value.weight", "attn.value.bias",
            "attn.out.weight", "attn.out.bias",
            "mlp_ln.weight", "mlp_ln.bias",
            "mlp.0.weight", "mlp.0.bias", "mlp.2.weight", "mlp.2.bias")]
    keys += ["ln_post.weight", "ln_post.bias"]
    return keys


def _shape(key, n_mels, d):
    if key == "conv1.weight":
        return (d, n_mels, 3)
    if key == "conv2.weight":
        return (d, d, 3)
    if key.endswith("mlp.0.weight"):
        return (4 * d, d)
    if key.endswith("mlp.0.bias"):
        return (4 * d,)
    if key.endswith("mlp.2.weight"):
        return (d, 4 * d)
    if key.endswith(".weight") and "attn." in key:
        return (d, d)
    return (d,)


def make_weights(model="tiny", seed=0, n_layer=None, std=0.02):
    """Random-init encoder weights: dict of ``"w." + name`` -> float32 array."""
    g = MODELS[model] if isinstance(model, str) else model
    n_mels, d = g["n_mels"], g["d"]
    n_layer = g["n_layer"] if n_layer is None else n_layer
    rng = np.random.default_rng(seed)
    s = np.float32(std)
    W = {}
    for k in weight_keys(n_layer):
        shp = _shape(k, n_mels, d)
        if k.endswith("_ln.weight") or k == "ln_post.weight":
            W["w." + k] = np.ones(shp, np.float32)
        elif k.endswith("_ln.bias") or k == "ln_post.bias":
            W["w." + k] = np.zeros(shp, np.float32)
        else:
            a = rng.standard_normal(shp, dtype=np.float32)
            a *= s
            W["w." + k] = a
    W["w.positional_embedding"] = sinusoids(g["n_ctx"], d)
    return W


def add_transposed(W):
    """The reference's derived ``*.weight_T`` (in, out) views of every 2-D
    Linear weight (npu_whisper_encoder.py:563-566)."""
    for k in [k for k in W if k.endswith(".weight") and W[k].ndim == 2
              and not k.endswith("_ln.weight")]:
        W[k[:-len("weight")] + "weight_T"] = np.ascontiguousarray(W[k].T)
    return W


def make_mel(n_mels=80, n_frames=3000, seed=0):
    """One synthetic log-mel [n_mels, n_frames]: N(-0.3, 0.5) clipped to [-1, 1.5]."""
    rng = np.random.default_rng(seed)
    m = rng.normal(-0.3, 0.5, (n_mels, n_frames)).astype(np.float32)
    return np.clip(m, -1.0, 1.5).astype(np.float32)


def make_mel_batch(batch, n_mels=80, n_frames=3000):
    """[batch, n_mels, n_frames], sample i drawn from seed i."""
    return np.stack([make_mel(n_mels, n_frames, seed=i) for i in range(batch)])


def rowop_inputs(seed=0):
    """The standalone row-op workloads (fp32 values; the kernels take them as
    bf16): LayerNorm [1500,1280] x~N(0,2), gamma~N(1,0.1), beta~N(0,0.1);
    GELU [1500,5120] x~N(0,3); softmax [30000,1500] logits~N(0,4)."""
    rng = np.random.default_rng(seed)
    return dict(
        ln_x=rng.normal(0, 2, (1500, 1280)).astype(np.float32),
        ln_gamma=rng.normal(1, 0.1, 1280).astype(np.float32),
        ln_beta=rng.normal(0, 0.1, 1280).astype(np.float32),
        gelu_x=rng.normal(0, 3, (1500, 5120)).astype(np.float32),
        sm_x=rng.normal(0, 4, (30000, 1500)).astype(np.float32),
    )
