"""The device-resident encoder forward (wxh_encoder_* in libwxhip.so).

`HipEncoder` uploads a whisper encoder's weights once (bf16 GEMM operands,
fp32 biases / LayerNorm / positional embedding) and runs mel -> features as
one hipGraph-captured stream of HIP kernels. It is what the drop-in
``encoder(W, mel, rt.matmul, ...)`` resolves to when the plugs are a HipRT's
own (see ``wxhip.encoder``), and what bench.py measures.
"""
import ctypes as C

import numpy as np

from . import _lib as L

STAGES = ("prep", "conv1", "conv2", "layernorm", "qkv", "attention", "out_proj",
          "fc1", "fc2", "ln_post")

_GELU = {"erf": L.WXH_GELU_ERF, "poly4": L.WXH_GELU_POLY4_RNE}


def geometry(W):
    """(n_mels, d_model, n_head, n_layer, n_ctx) read off a weight dict, the
    way npu_whisper_encoder.py:568-573 does (n_head = d / 64)."""
    n_layer = 1 + max(int(k.split(".")[2]) for k in W if k.startswith("w.blocks."))
    d, n_mels, _ = W["w.conv1.weight"].shape
    n_ctx = W["w.positional_embedding"].shape[0]
    return n_mels, d, d // 64, n_layer, n_ctx


def weight_names(n_layer):
    names = ["conv1.weight", "conv1.bias", "conv2.weight", "conv2.bias",
             "positional_embedding", "ln_post.weight", "ln_post.bias"]
    for i in range(n_layer):
        p = f"blocks.{i}."
        names += [p + s for s in (
            "attn_ln.weight", "attn_ln.bias", "attn.query.weight", "attn.query.bias",
            "attn.key.weight", "attn.value.weight", "attn.value.bias",
            "attn.out.weight", "attn.out.bias", "mlp_ln.weight", "mlp_ln.bias",
            "mlp.0.weight", "mlp.0.bias", "mlp.2.weight", "mlp.2.bias")]
    return names


class HipEncoder:
    """Whisper encoder on one GPU: weights resident, forward as a hipGraph."""

    def __init__(self, dev, W, n_layer=None, mlp_gelu="erf", graph=True, int8=False,
                 conv_gelu="erf"):
        n_mels, d, n_head, nl, n_ctx = geometry(W)
        self.dev = dev
        self.n_mels, self.d_model, self.n_head, self.n_ctx = n_mels, d, n_head, n_ctx
        self.n_layer = nl if n_layer is None else n_layer
        if not 0 <= self.n_layer <= nl:
            raise ValueError(f"n_layer={self.n_layer} but the weights have {nl} blocks")
        for name, v in (("mlp_gelu", mlp_gelu), ("conv_gelu", conv_gelu)):
            if v not in _GELU:
                raise ValueError(f"{name} must be one of {sorted(_GELU)}")
        self.mlp_gelu, self.conv_gelu = mlp_gelu, conv_gelu
        dims = L.EncoderDims(n_mels, d, n_head, self.n_layer, n_ctx, _GELU[mlp_gelu],
                             _GELU[conv_gelu])
        h = C.c_void_p()
        L.call("wxh_encoder_create", dev.handle, C.byref(dims), C.byref(h))
        self._h = h
        # int8: int8 copies of the GEMM weights are made while they upload
        # (per output channel, from the fp32 values), and the forward runs
        # the int8 GEMM path (wxh_encoder_set_int8); set_int8(False) goes
        # back to bf16 with the same weights
        self.int8_capable = bool(int8)
        self.int8 = False
        if int8:
            L.call("wxh_encoder_enable_int8", self._h)
        self.load_weights(W)
        if int8:
            self.set_int8(True)
        if not graph:
            L.call("wxh_encoder_set_graph", self._h, 0)

    def set_int8(self, on):
        """Switch the forward between the int8 and the bf16 GEMM path (int8
        needs the encoder built with int8=True)."""
        L.call("wxh_encoder_set_int8", self._h, int(bool(on)))
        self.int8 = bool(on)

    def load_weights(self, W):
        for name in weight_names(self.n_layer):
            a = np.ascontiguousarray(W["w." + name], dtype=np.float32)
            shape = (C.c_int64 * a.ndim)(*a.shape)
            L.call("wxh_encoder_set_weight", self._h, ("w." + name).encode(),
                   a.ctypes.data_as(C.c_void_p), shape, a.ndim)
        L.call("wxh_encoder_ready", self._h)

    def set_graph(self, enabled):
        L.call("wxh_encoder_set_graph", self._h, int(bool(enabled)))

    def ctx_len(self, n_frames):
        return (n_frames - 1) // 2 + 1

    def forward(self, mel, out=None):
        """mel: fp32 torch tensor on the device, [B, n_mels, T] or [n_mels, T]
        -> fp32 [B, ctx, d] (or [ctx, d])."""
        import torch
        squeeze = mel.dim() == 2
        m = mel[None] if squeeze else mel
        if m.dtype != torch.float32 or m.device != self.dev.device or m.shape[1] != self.n_mels:
            raise ValueError(f"mel must be fp32 [B, {self.n_mels}, T] on {self.dev.device}")
        m = m.contiguous()
        B, _, T = m.shape
        ctx = self.ctx_len(T)
        if out is None:
            out = torch.empty(B, ctx, self.d_model, dtype=torch.float32, device=self.dev.device)
        L.call("wxh_encoder_forward", self._h, C.c_void_p(m.data_ptr()), B, T,
               C.c_void_p(out.data_ptr()), self.dev.stream())
        return out[0] if squeeze else out

    @classmethod
    def from_file(cls, dev, path, **kw):
        """Weights from a dump_ref.py ``.npz`` or an openai-whisper checkpoint
        (wxhip.weights), uploaded once as device bf16."""
        from . import weights
        return cls(dev, weights.load(path), **kw)

    def forward_audio(self, audio, out=None):
        """16 kHz fp32 audio on the device, [B, n_samples] or [n_samples]
        (30 s windows: 480000 samples) -> features, with the log-mel front end
        on the GPU as well (Device.log_mel with this model's n_mels)."""
        mel = self.dev.log_mel(audio, self.n_mels)
        return self.forward(mel, out=out)

    def forward_numpy(self, mel):
        """Host fp32 mel [B, n_mels, T] or [n_mels, T] -> host fp32 features."""
        m = np.ascontiguousarray(mel, dtype=np.float32)
        squeeze = m.ndim == 2
        if squeeze:
            m = m[None]
        B, nm, T = m.shape
        if nm != self.n_mels:
            raise ValueError(f"mel has {nm} bins, the weights want {self.n_mels}")
        out = np.empty((B, self.ctx_len(T), self.d_model), np.float32)
        L.call("wxh_encoder_forward_host", self._h, m.ctypes.data_as(C.c_void_p), B, T,
               out.ctypes.data_as(C.c_void_p))
        return out[0] if squeeze else out

    def profile(self, mel, out=None):
        """One un-graphed forward; returns {stage: device ms} timed with HIP
        events on the library stream."""
        import torch
        m = (mel[None] if mel.dim() == 2 else mel).contiguous()
        B, _, T = m.shape
        if out is None:
            out = torch.empty(B, self.ctx_len(T), self.d_model, dtype=torch.float32,
                              device=self.dev.device)
        torch.cuda.synchronize(self.dev.device)
        ms = (C.c_float * len(STAGES))()
        L.call("wxh_encoder_profile", self._h, C.c_void_p(m.data_ptr()), B, T,
               C.c_void_p(out.data_ptr()), ms, len(STAGES))
        return dict(zip(STAGES, [float(v) for v in ms]))

    def close(self):
        if getattr(self, "_h", None):
            L.load().wxh_encoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
